// Helpers shared by the SSD prefill kernels and their backward: the dt prologue, the in-segment decay
// scan and the fragment-native order of per-(batch, chunk, head) states in the workspaces.
#pragma once

#include "common.h"
#include "launch.h"

namespace mh {

constexpr int HD = 64;               // headdim handled by the SSD kernels
// Two-pass prefill: most chunks whose entering states the scan sums itself from the chunk states (more
// chunks get them from ssd_state_pass_kernel).
constexpr int LB_MAX = 8;

__host__ __device__ __forceinline__ size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// dt <- clamp(softplus?(dt + bias), dt_min, dt_max) per the flags.
__device__ __forceinline__ float process_dt(const SsdParams& p, float dt, float bias) {
  dt += bias;
  if (p.dt_softplus) dt = softplus_f(dt);
  if (p.has_dt_limit) dt = fminf(fmaxf(dt, p.dt_min), p.dt_max);
  return dt;
}

// In-segment decay of one head (lane = token; tokens at or past c1 have dt = 0):
// returns cs_t, the inclusive cumulative log-decay.
__device__ __forceinline__ float seg_decay(const SsdParams& p, float dtraw, float bias, float Ah, int t, int c1,
                                           float& dtv) {
  dtv = (t < c1) ? process_dt(p, dtraw, bias) : 0.f;
  return wave_incl_scan_dpp(Ah * dtv);
}

// A state of HD x N values is stored in fragment-native order: 32x32 tile (nt, pt) -- rows n = 32 nt..,
// columns p = 32 pt.. -- as an accumulator tile (lane = column p % 32, element r = row acc_row(half, r)) in a
// block of 64 x 16 values.  fp32: 16 consecutive values per lane; offset (elements) of tile (nt, pt)'s block of
// lane l:
__device__ __forceinline__ int frag_off(int nt, int pt, int l) { return ((nt * 2 + pt) * 64 + l) * 16; }
// bf16 states: piece q (accumulator elements 8 q .. 8 q + 7) of lane l in block (nt, pt) -- the block's 64 x 16
// elements as two halves of 64 lanes x 8, so that one wave-wide 16-byte access is 1 KB contiguous.
__device__ __forceinline__ int frag_off_bf(int nt, int pt, int l, int q) {
  return (nt * 2 + pt) * 1024 + q * 512 + l * 8;
}

// Row permutation of the two-pass prefill's states: within each 16-row group, 4-row blocks 1 and 2 are
// swapped, so that accumulator row 16 c + KSET(half, j) holds state n = 16 c + 8 half + j (the state rows a
// KSET-ordered read-out fragment meets in natural column order).
__host__ __device__ __forceinline__ int state_row_perm(int r) {
  const int m = (r >> 2) & 3;
  return (r & ~12) | ((((m & 1) << 1) | (m >> 1)) << 2);
}

// Workspace element e (fragment-native order; bf: the frag_off_bf layout) <-> canonical state index p * N + n
// (perm: rows permuted by state_row_perm, the two-pass prefill's order).
__device__ __forceinline__ int canon_index(int e, int N, bool perm, bool bf) {
  const int r = bf ? ((e >> 9) & 1) * 8 + (e & 7) : e & 15;
  const int lane = bf ? (e >> 3) & 63 : (e >> 4) & 63, tile = e >> 10;
  const int pt = tile & 1, nt = tile >> 1;
  const int row = acc_row(lane >> 5, r);
  return (32 * pt + (lane & 31)) * N + 32 * nt + (perm ? state_row_perm(row) : row);
}

}  // namespace mh
