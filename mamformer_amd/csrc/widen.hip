// Element-wise helpers with which the C ABI runs sizes the scan kernels do not
// tile natively as compositions of sizes they do (capi.hip):
//   * SSD state sizes below 64 (or between 64 and 128): B, C and the state
//     zero-padded to 64 (128) columns.  Padded state columns receive B = 0 and
//     start at zero, so they stay zero, and C = 0 keeps them out of y; the
//     gradients of the real columns are those of the unpadded problem.
//   * SSD state sizes above 128: two runs over the 128-column halves of B, C
//     and the state (the second zero-padded).  The recurrence is independent
//     per state column given dt and A, so y = y(half 0) + y(half 1) with D
//     applied in one of them, the gate after the sum, and the gradients of
//     dt, A, dt_bias and x summed over the halves.
// col_copy moves a column window of a 3-level row set (zero-filling columns
// beyond the source window); row_add adds one such row set into another,
// optionally multiplying by silu(gate) as it stores.  gate_fwd / gate_bwd are
// the block's output gate y * silu(z) and its gradient for the training path,
// 8 elements (16 bytes of bf16) per thread and step.
#include "common.h"
#include "launch.h"

namespace mh {

namespace {

template <typename T>
__global__ __launch_bounds__(256) void col_copy_kernel(ColCopy c) {
  const int64_t total = c.d0 * c.d1 * c.d2 * c.ncols;
  const T* src = reinterpret_cast<const T*>(c.src);
  T* dst = reinterpret_cast<T*>(c.dst);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t col = i % c.ncols, row = i / c.ncols;
    const int64_t i2 = row % c.d2, r01 = row / c.d2;
    const int64_t i1 = r01 % c.d1, i0 = r01 / c.d1;
    T v = from_f32<T>(0.f);
    if (col < c.nvalid) v = src[i0 * c.s0 + i1 * c.s1 + i2 * c.s2 + c.scol0 + col];
    dst[i0 * c.t0 + i1 * c.t1 + i2 * c.t2 + c.tcol0 + col] = v;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void row_add_kernel(RowAdd a) {
  const int64_t total = a.d0 * a.d1 * a.d2 * a.ncols;
  T* dst = reinterpret_cast<T*>(a.dst);
  const T* src = reinterpret_cast<const T*>(a.src);
  const T* gate = reinterpret_cast<const T*>(a.gate);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t col = i % a.ncols, row = i / a.ncols;
    const int64_t i2 = row % a.d2, r01 = row / a.d2;
    const int64_t i1 = r01 % a.d1, i0 = r01 / a.d1;
    const int64_t od = i0 * a.t0 + i1 * a.t1 + i2 * a.t2 + col;
    float v = to_f32(dst[od]) + to_f32(src[i0 * a.s0 + i1 * a.s1 + i2 * a.s2 + col]);
    if (gate) v *= silu_f(to_f32(gate[i0 * a.g0 + i1 * a.g1 + i2 * a.g2 + col]));
    dst[od] = from_f32<T>(v);
  }
}

// Row r of a (d0, d1, d2) row set with strides (s0, s1, s2): its offset.
__device__ __forceinline__ int64_t row_off(int64_t r, int64_t d1, int64_t d2, int64_t s0, int64_t s1, int64_t s2) {
  const int64_t i2 = r % d2, r01 = r / d2;
  return (r01 / d1) * s0 + (r01 % d1) * s1 + i2 * s2;
}

template <typename T> struct Vec8;
template <> struct Vec8<bf16> {
  __device__ static void load(const bf16* p, float (&v)[8]) {
    const bf16x8 b = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)b[j];
  }
  __device__ static void store(bf16* p, const float (&v)[8]) {
    bf16x8 b;
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (bf16)v[j];
    *reinterpret_cast<bf16x8*>(p) = b;
  }
};
template <> struct Vec8<float> {
  __device__ static void load(const float* p, float (&v)[8]) {
    const f32x4 a = reinterpret_cast<const f32x4*>(p)[0], b = reinterpret_cast<const f32x4*>(p)[1];
#pragma unroll
    for (int j = 0; j < 4; ++j) { v[j] = a[j]; v[4 + j] = b[j]; }
  }
  __device__ static void store(float* p, const float (&v)[8]) {
    reinterpret_cast<f32x4*>(p)[0] = f32x4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<f32x4*>(p)[1] = f32x4{v[4], v[5], v[6], v[7]};
  }
};

template <typename T, bool BWD>
__global__ __launch_bounds__(256) void gate_kernel(GateParams a) {
  const int64_t per = a.ncols / 8, total = a.d0 * a.d1 * a.d2 * per;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / per, c = 8 * (i % per);
    float y[8], z[8], o[8];
    Vec8<T>::load(reinterpret_cast<const T*>(a.y) + row_off(r, a.d1, a.d2, a.y0, a.y1, a.y2) + c, y);
    Vec8<T>::load(reinterpret_cast<const T*>(a.z) + row_off(r, a.d1, a.d2, a.z0, a.z1, a.z2) + c, z);
    if constexpr (!BWD) {
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = y[j] * silu_f(z[j]);
    } else {
      float g[8], dz[8];
      Vec8<T>::load(reinterpret_cast<const T*>(a.g) + row_off(r, a.d1, a.d2, a.g0, a.g1, a.g2) + c, g);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float sg = __builtin_amdgcn_rcpf(1.f + __expf(-z[j]));       // sigmoid (1 ulp reciprocal)
        o[j] = g[j] * z[j] * sg;
        dz[j] = g[j] * y[j] * (sg * (1.f + z[j] * (1.f - sg)));
      }
      Vec8<T>::store(reinterpret_cast<T*>(a.dz) + row_off(r, a.d1, a.d2, a.dz0, a.dz1, a.dz2) + c, dz);
    }
    Vec8<T>::store(reinterpret_cast<T*>(a.out) + row_off(r, a.d1, a.d2, a.o0, a.o1, a.o2) + c, o);
  }
}

unsigned blocks_for(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

hipError_t launch_gate(const GateParams& a, bool backward, hipStream_t st) {
  const int64_t total = a.d0 * a.d1 * a.d2 * (a.ncols / 8);
  if (total <= 0) return hipSuccess;
  const unsigned nb = blocks_for(total);
  if (a.es == 4) {
    if (backward) gate_kernel<float, true><<<nb, 256, 0, st>>>(a);
    else gate_kernel<float, false><<<nb, 256, 0, st>>>(a);
  } else {
    if (backward) gate_kernel<bf16, true><<<nb, 256, 0, st>>>(a);
    else gate_kernel<bf16, false><<<nb, 256, 0, st>>>(a);
  }
  return hipGetLastError();
}

hipError_t launch_col_copy(const ColCopy& c, hipStream_t st) {
  const int64_t total = c.d0 * c.d1 * c.d2 * c.ncols;
  if (total <= 0) return hipSuccess;
  if (c.es == 4)
    col_copy_kernel<float><<<blocks_for(total), 256, 0, st>>>(c);
  else
    col_copy_kernel<bf16><<<blocks_for(total), 256, 0, st>>>(c);
  return hipGetLastError();
}

hipError_t launch_row_add(const RowAdd& a, hipStream_t st) {
  const int64_t total = a.d0 * a.d1 * a.d2 * a.ncols;
  if (total <= 0) return hipSuccess;
  if (a.es == 4)
    row_add_kernel<float><<<blocks_for(total), 256, 0, st>>>(a);
  else
    row_add_kernel<bf16><<<blocks_for(total), 256, 0, st>>>(a);
  return hipGetLastError();
}

}  // namespace mh
