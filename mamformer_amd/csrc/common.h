// Shared device helpers for the gfx950 scan kernels: element conversion,
// 32x32 MFMA tiles (bf16 and fp32 operand flavours) and wave primitives.
//
// Register layout of one 32x32 fp32 accumulator tile (f32x16 per lane), as the
// CDNA3/CDNA4 32x32 MFMA family writes it:
//     lane l, element r  ->  row = 8*(r/4) + 4*(l/32) + (r%4),  col = l%32
// Operand fragments (8 values per lane, one 32x32x16 step):
//     A[row][k]: lane l holds row l%32,  B[k][col]: lane l holds col l%32,
// and the 8 k-values a lane holds are addressed by (half = l/32, j = 0..7).
// The contraction runs over (half, j) identically for A and B, so any
// bijection (half, j) -> k is a valid "k-set" as long as both operands use
// it.  The kernels use the *accumulator-derived* k-set
//     KSET(half, j) = (j < 4) ? 4*half + j : 8 + 4*half + (j - 4)     (within a 16-wide k-step)
// which is exactly the set of rows an accumulator tile gives a lane for one
// 16-row half of the tile.  That lets an fp32 accumulator tile be fed back as
// an MFMA operand (after conversion) with no data movement.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

typedef __bf16 bf16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) __bf16 bf16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16 v) { return (float)v; }
template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float v) { return (bf16)v; }

// KSET position of element j of a fragment held by lane-half `half`.
__device__ __forceinline__ int kset(int half, int j) {
  return (j < 4) ? (4 * half + j) : (8 + 4 * half + (j - 4));
}

// ---------------------------------------------------------------- MFMA tiles
// Fragment of 8 operand values in MFMA input precision.
template <typename TM> struct Frag;
template <> struct Frag<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void set(int j, float x) { v[j] = (bf16)x; }
  __device__ __forceinline__ float get(int j) const { return (float)v[j]; }
};
template <> struct Frag<float> {
  float v[8];
  __device__ __forceinline__ void set(int j, float x) { v[j] = x; }
  __device__ __forceinline__ float get(int j) const { return v[j]; }
};

// acc += A(32x16) * B(16x32) for one k-step.
__device__ __forceinline__ f32x16 mma(const Frag<bf16>& a, const Frag<bf16>& b, f32x16 acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a.v, b.v, acc, 0, 0, 0);
}
// fp32 operands: eight 32x32x2 steps, step j consuming element j of each half.
__device__ __forceinline__ f32x16 mma(const Frag<float>& a, const Frag<float>& b, f32x16 acc) {
#pragma unroll
  for (int j = 0; j < 8; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a.v[j], b.v[j], acc, 0, 0, 0);
  return acc;
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// Row of accumulator element r for lane-half `half` (see header comment).
__device__ __forceinline__ int acc_row(int half, int r) { return 8 * (r >> 2) + 4 * half + (r & 3); }

// Operand fragment for k-step `c` (0 or 1) taken from an accumulator tile:
// element j of the fragment is accumulator row 16*c + KSET(half, j).
template <typename TM>
__device__ __forceinline__ Frag<TM> acc_to_frag(const f32x16& acc, int c) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, acc[8 * c + j]);
  return f;
}
// Same with a per-element scale.
template <typename TM>
__device__ __forceinline__ Frag<TM> acc_to_frag_scaled(const f32x16& acc, int c, float s) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, acc[8 * c + j] * s);
  return f;
}

// ---------------------------------------------------------------- wave helpers
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
// v from the lane the DPP control CTRL selects (rows in ROWS; every lane of the selected rows active).
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, false));
}
// The lane index recomputed where it is used (v_mbcnt in a volatile asm): address arithmetic built on it is not
// hoisted out of loops, where it would hold registers for the whole loop.
__device__ __forceinline__ int lane_id_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
// Wave index within the workgroup, in a scalar register (wave-uniform for the compiler).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ float wave_incl_scan(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (l >= off) v += o;
  }
  return v;
}
// Same scan on the DPP crossbar (row shifts within 16-lane rows, then the row
// broadcasts of lanes 15 and 31): six dependent VALU ops instead of six LDS
// permutes.
__device__ __forceinline__ float wave_incl_scan_dpp(float v) {
  int iv;
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false);   // row_shr:1
  v += __int_as_float(iv);
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, false);   // row_shr:2
  v += __int_as_float(iv);
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, false);   // row_shr:4
  v += __int_as_float(iv);
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, false);   // row_shr:8
  v += __int_as_float(iv);
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xa, 0xf, false);   // row_bcast:15 -> rows 1, 3
  v += __int_as_float(iv);
  iv = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xc, 0xf, false);   // row_bcast:31 -> rows 2, 3
  v += __int_as_float(iv);
  return v;
}

// v of lane `lane` (wave-uniform) in every lane: v_readlane, no LDS permute.
__device__ __forceinline__ float lane_val(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
// v of lane 32 x + lane % 32 (x = 0 or 1, wave-uniform) in every lane, by v_permlane32_swap.
__device__ __forceinline__ float from_half(float v, int x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(x ? r[1] : r[0]);
}
// v of this lane plus v of the lane 32 away, the same sum in both lanes (v_permlane32_swap: no LDS permute).
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A wave's 16 floats per lane parked in LDS as four planes of 16-byte pieces (plane k holds elements 4k .. 4k + 3
// of every lane, lanes contiguous): each wave-wide 16-byte access is 1 KB contiguous, free of bank conflicts (a
// 64-byte lane stride puts four lanes of every 16 on one bank).
struct AccPark {
  f32x4 p[4][64];
};
__device__ __forceinline__ void park_acc(AccPark& d, const float (&v)[16], int lane) {
#pragma unroll
  for (int k = 0; k < 4; ++k) d.p[k][lane] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
}
__device__ __forceinline__ void park_acc(AccPark& d, const f32x16& v, int lane) {
#pragma unroll
  for (int k = 0; k < 4; ++k) d.p[k][lane] = f32x4{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
}
__device__ __forceinline__ f32x16 unpark_acc(const AccPark& d, int lane) {
  f32x16 v;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f32x4 q = d.p[k][lane];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[4 * k + j] = q[j];
  }
  return v;
}

// Sum over each group of 4 lanes (quad permutes on the DPP crossbar), the same in the 4 lanes.
__device__ __forceinline__ float sum_quad(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad_perm 1,0,3,2
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad_perm 2,3,0,1
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fminf(v, __shfl_xor(v, off, 64));
  return v;
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations,
// then s_barrier.  __syncthreads() also carries a workgroup release fence, which
// on gfx950 waits for every outstanding global load and store (vmcnt(0)) --
// including asynchronous prefetches meant to overlap the compute that follows.
// Callers that need prefetched data (global_load_lds) wait for vmcnt themselves.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// softplus with PyTorch's default threshold (x > 20 -> x): log(1 + e^x).  For e = e^x < 1/16 the
// log1p series e - e^2/2 + ... + e^7/7 (truncation below e^8/8, i.e. < 4e-10 relative); above, 1 + e
// is formed with relative rounding error 6e-8 against a logarithm >= 0.06.
__device__ __forceinline__ float softplus_f(float x) {
  if (x > 20.f) return x;
  const float e = __expf(x);
  if (e < 0.0625f) {
    float s = 1.f / 7.f;
    s = 1.f / 6.f - e * s;
    s = 1.f / 5.f - e * s;
    s = 1.f / 4.f - e * s;
    s = 1.f / 3.f - e * s;
    s = 1.f / 2.f - e * s;
    s = 1.f - e * s;
    return e * s;
  }
  return __logf(1.f + e);
}

// silu(x) = x / (1 + e^{-x}), the quotient through the hardware reciprocal (v_rcp_f32, 1 ulp) rather than an
// IEEE division sequence; e^{-x} overflowing to +inf gives -0 (the limit) for very negative x.
__device__ __forceinline__ float silu_f(float x) { return x * __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// sigmoid(x) = 1 / (1 + e^{-x}) through the same reciprocal (0 for e^{-x} = +inf).
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

}  // namespace mh
