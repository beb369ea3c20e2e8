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
// optionally multiplying by silu(gate) as it stores.
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

unsigned blocks_for(int64_t total) {
  const int64_t b = (total + 255) / 256;
  return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

}  // namespace

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
