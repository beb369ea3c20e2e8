// Helpers shared by the SSD prefill kernels and their backward: the dt prologue, the in-segment decay
// scan and the fragment-native order of per-(batch, chunk, head) states in the workspaces.
#pragma once

#include "common.h"
#include "launch.h"

namespace mh {

constexpr int HD = 64;               // headdim handled by the SSD kernels

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
// columns p = 32 pt.. -- as an accumulator tile (lane = column p % 32, element r = row acc_row(half, r)),
// 16 consecutive values per lane.  Offset (elements) of tile (nt, pt)'s block of lane l:
__device__ __forceinline__ int frag_off(int nt, int pt, int l) { return ((nt * 2 + pt) * 64 + l) * 16; }

// Workspace element e (fragment-native order) <-> canonical state index p * N + n.
__device__ __forceinline__ int canon_index(int e, int N) {
  const int r = e & 15, lane = (e >> 4) & 63, tile = e >> 10;
  const int pt = tile & 1, nt = tile >> 1;
  return (32 * pt + (lane & 31)) * N + 32 * nt + acc_row(lane >> 5, r);
}

}  // namespace mh
