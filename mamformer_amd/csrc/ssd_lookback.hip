// Mamba-2 SSD chunked-scan prefill for gfx950, bf16 I/O, in two passes over the sequence.
//
// Recurrence (per batch b, head h with group g = h / (H/G), channel p, state n):
//     h_t = exp(A_h dt_t) h_{t-1} + dt_t x_t[p] B_t[g, n]
//     y_t[p] = sum_n C_t[g, n] h_t[p, n] + D x_t[p]
// -- the reference's selective_scan (mamformer/layers/mamba2.py:84-126) in the per-head SSD form, with an
// optional initial state and the final state returned for the decode cache.
//
// Pass 1, ssd_lb_state_kernel, one workgroup per (chunk, batch, block of heads): the chunk-local state
//     S_k[p, n] = sum_{s in k} exp(sum_{s < tau in k} A dt_tau) dt_s x_s[p] B_s[n]
// and the chunk's total log-decay T_k.  The chunk is walked from its last 64-token segment to its first, so
// every decay factor is taken relative to the chunk end and is at most 1: the accumulators never need
// rescaling.  The per-token weight w_s multiplies x on the MFMA unit (xs = diag(w) x, x read transposed out
// of LDS with ds_read_b64_tr_b16).  S_k leaves in bf16, in MFMA fragment order with its state rows permuted
// (state_row_perm), the order in which the scan's read-out meets C in natural column order.
//
// Pass 2, ssd_lb_scan_kernel, same workgroups: the entering state
//     H_k = sum_{j<k} exp(T_{j+1} + .. + T_{k-1}) S_j  +  exp(T_0 + .. + T_{k-1}) h0
// is summed straight from pass 1's chunk states (a look-back over at most LB_MAX - 1 predecessors; longer
// sequences get the entering states from ssd_state_pass_kernel between the passes), then the chunk is walked
// forward in 64-token segments with the running state in MFMA accumulators, carried lazily as
// H_true = e^kappa H so that one scaled operand xs_s = e^{-kappa-cs_s} dt_s x_s serves both the state update
// H += B^T xs and the intra-segment term (cs_t the in-segment inclusive cumulative log-decay):
//     y_t = e^{kappa + cs_t} (C_t H^T + sum_{s<=t} (C_t . B_s) xs_s) + D x_t,   kappa += cs_end.
// The three masked (C B^T) tiles of a segment are formed once per workgroup and shared through LDS.  A
// segment whose own decay range exceeds LB_FACT_RANGE takes an exact per-element path (wave-uniform branch).
//
// Work split (both passes): a workgroup owns HG heads of one group (pass 1 on chunks of at most
// LB_STATE_SHORT tokens: two heads), 2 / PH waves per head; a wave's state is PH of its head's two 32-column
// halves of P as N/32 accumulator tiles each (rows n, columns p).  With PH = 1 (LB_PH, two waves per head,
// two waves per SIMD) every B / C operand fragment a wave reads from LDS feeds one MFMA; PH = 2 (one wave per
// head, both halves from each fragment) needs ~500 registers and one wave per SIMD, and measured slower.  Every segment's tiles (x, B, C, dt) are fetched
// straight into LDS (global_load_lds) ahead of use, in the Sub64 layout (tiles.h): every LDS access of the
// loops is one lane offset (a few per kernel) plus an immediate, the stage being a compile-time index (the
// segment loop is unrolled by the number of stages).
#include <type_traits>

#include "common.h"
#include "launch.h"
#include "ssd_shared.h"
#include "tiles.h"

namespace mh {

namespace {

constexpr float LB_FACT_RANGE = 60.f;   // max exponent of an operand scale factor (pass 2)
constexpr size_t LB_LDS_BYTES = 160 * 1024;

template <int v> using IC = std::integral_constant<int, v>;

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// ds_read_b64_tr_b16: within each 16-lane group the four lanes 4k..4k+3 name a row of 16 consecutive 16-bit
// elements (4 each, 8-byte aligned) and lane j of the group receives element j of rows k = 0..3.
__device__ __forceinline__ i16x4 ds_tr16(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// Lane offsets (elements) of the access patterns, each valid for every sub-tile and token block.
struct LaneOffs {
  int tr[2];     // transposed read: rows 4 half + (lane & 15) / 4 (+ 8 for [1]), columns 16 ((lane >> 4) & 1) + 4 (lane & 3)
  int trp[2];    // the same with the column pieces 4-7 and 8-11 of each 16 swapped (lane j gets column state_row_perm(j))
  int row[2];    // row fragment: row lane % 32, columns 16 c + 8 half, [c]
  int piece[4];  // 8-byte row pieces: row lane % 32, columns 8 q + 4 half, [q]
};
__device__ __forceinline__ LaneOffs lane_offs(int l) {
  const int half = l >> 5, l32 = l & 31, i = l & 15;
  const int tc = 16 * ((l >> 4) & 1) + 4 * (i & 3);
  const int tcp = 16 * ((l >> 4) & 1) + 4 * (((i & 1) << 1) | ((i >> 1) & 1));
  LaneOffs o;
#pragma unroll
  for (int e = 0; e < 2; ++e) o.tr[e] = Sub64::off(4 * half + (i >> 2) + 8 * e, tc);
#pragma unroll
  for (int e = 0; e < 2; ++e) o.trp[e] = Sub64::off(4 * half + (i >> 2) + 8 * e, tcp);
#pragma unroll
  for (int c = 0; c < 2; ++c) o.row[c] = Sub64::off(l32, 16 * c + 8 * half);
#pragma unroll
  for (int q = 0; q < 4; ++q) o.piece[q] = Sub64::off(l32, 8 * q + 4 * half);
  return o;
}

// MFMA operand fragment read transposed from a Sub64 sub-tile: the lane's column is lane % 32 (state_row_perm
// of it with the trp offsets) and its 8 k-values are the tokens row0 + KSET(half, 0..7) (row0 % 16 == 0).  The
// same registers serve as an A operand (row = tile column) or a B operand (column = tile column).
__device__ __forceinline__ Frag<bf16> tr_frag(const bf16* sub, int row0, const int (&off)[2]) {
  const i16x4 a = ds_tr16(sub + row0 * Sub64::W + off[0]);
  const i16x4 b = ds_tr16(sub + row0 * Sub64::W + off[1]);
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  return f;
}
// Row fragment: row row0 + lane % 32 (row0 % 32 == 0), the 8 consecutive columns 16 c + 8 half of a sub-tile.
__device__ __forceinline__ Frag<bf16> row_frag64(const bf16* sub, int row0, int c, const LaneOffs& lo) {
  Frag<bf16> f;
  f.v = *reinterpret_cast<const bf16x8*>(sub + row0 * Sub64::W + lo.row[c]);
  return f;
}

// Diagonal A-operand fragments (k-steps c = 0, 1) of one 32-token block, D[s][s'] = w_s [s == s'].  Lane
// (row s = lane % 32, half) holds its diagonal element only in k-step s >> 4 at position
// (s & 3) + 4 ((s >> 3) & 1), and only when half == (s >> 2) & 1 (the KSET order); the masks below select
// that 16-bit slot.
struct DiagMask {
  uint32_t m[2][4];
};
__device__ __forceinline__ DiagMask diag_mask(int l) {
  const int s = l & 31, half = l >> 5;
  const bool on = half == ((s >> 2) & 1);
  const int cc = s >> 4, jj = (s & 3) + 4 * ((s >> 3) & 1);
  DiagMask d;
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      d.m[c][q] = (on && c == cc && q == (jj >> 1)) ? ((jj & 1) ? 0xffff0000u : 0x0000ffffu) : 0u;
  return d;
}
__device__ __forceinline__ void diag_frags(float w, const DiagMask& dm, Frag<bf16> (&f)[2]) {
  const uint32_t b = (uint32_t)__builtin_bit_cast(uint16_t, (bf16)w);
  const uint32_t d = b | (b << 16);
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    u32x4 v;
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = d & dm.m[c][q];
    f[c].v = __builtin_bit_cast(bf16x8, v);
  }
}

// The value of lane (32 * st + lane % 32) in every lane: [0] for st = 0, [1] for st = 1.
__device__ __forceinline__ void halves(float v, float (&o)[2]) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  o[0] = __uint_as_float(r[0]);
  o[1] = __uint_as_float(r[1]);
}

// Workgroup -> (chunk k, chain = batch * (H / HG) + head block).  Workgroups are dealt to the 8 XCDs
// round-robin by index; when the chains split evenly over them, XCD x runs every chunk of the consecutive
// chains [x cpx, (x + 1) cpx): the scan finds its predecessors' chunk states in that XCD's L2, and the head
// blocks sharing a group's B and C tiles (consecutive chains) read them through as few L2s as possible.
__device__ __forceinline__ void lb_block(int nchunks, int nchains, int& k, int& chain) {
  const int i = blockIdx.x;
  if ((nchains & 7) == 0) {
    const int cpx = nchains >> 3, s = i >> 3;
    chain = (i & 7) * cpx + s % cpx;
    k = s / cpx;
  } else {
    k = i % nchunks;
    chain = i / nchunks;
  }
}

// xs = diag(w) x for the wave's PH 64 x 32 halves of its head (Sub64 sub-tiles at x + ph ELEMS): B-operand
// fragments xa[ph][2 * st + c] (k = token of block st, k-step c; column = p).  wb[st] = w of token
// 32 st + lane % 32.
template <int PH>
__device__ __forceinline__ void scaled_x(const bf16* x, const float (&wb)[2], const DiagMask& dm, const LaneOffs& lo,
                                         Frag<bf16> (&xa)[PH][4]) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    Frag<bf16> dg[2];
    diag_frags(wb[st], dm, dg);
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < 2; ++c) acc = mma(dg[c], tr_frag(x + ph * Sub64::ELEMS, 32 * st + 16 * c, lo.tr), acc);
      xa[ph][2 * st] = acc_to_frag<bf16>(acc, 0);
      xa[ph][2 * st + 1] = acc_to_frag<bf16>(acc, 1);
    }
  }
}

// H[ph][n][p] += sum_s B^T[n][s] xs[ph][s][p] over the segment's 64 tokens, B^T read transposed from the B tile
// with the state rows in state_row_perm order; the fragments of tile nt + 1 are requested before tile nt's
// MFMAs, and issue(nt) (global -> LDS loads of a later segment) runs between them, so that the loads queue at
// the memory unit while the matrix unit works.
struct NoIssue {
  __device__ void operator()(int) const {}
};
template <int N, int PH, typename Issue = NoIssue>
__device__ __forceinline__ void lb_state_update(f32x16 (&H)[PH][N / 32], const bf16* btile,
                                                const Frag<bf16> (&xa)[PH][4], const LaneOffs& lo,
                                                const Issue& issue = Issue()) {
  Frag<bf16> cur[4], nxt[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) cur[c] = tr_frag(btile, 16 * c, lo.trp);
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt) {
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) nxt[c] = tr_frag(btile + (nt + 1) * Sub64::ELEMS, 16 * c, lo.trp);
    }
    issue(nt);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int ph = 0; ph < PH; ++ph) H[ph][nt] = mma(cur[c], xa[ph][c], H[ph][nt]);
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) cur[c] = nxt[c];
    }
  }
}

// Read-out of the state entering the segment, Y^T[ph][tt][p][t] = sum_n H[ph][p][n] C[32 tt + t][n] (C as natural
// row fragments: the permuted state rows meet natural column order in the KSET-ordered accumulator fragments),
// fused per 32-row state tile with the state update H += B^T xs; the fragments of tile nt + 1 are requested
// before tile nt's MFMAs.
template <int N, int PH>
__device__ __forceinline__ void readout(f32x16 (&H)[PH][N / 32], f32x16 (&Y)[PH][2], const bf16* ctile,
                                        const bf16* btile, const Frag<bf16> (&xa)[PH][4], const LaneOffs& lo) {
  Frag<bf16> cc[4], cb[4], nc[4], nb[4];   // C: [2 c + tt], B: [c]
  auto load = [&](int nt, Frag<bf16> (&fc)[4], Frag<bf16> (&fb)[4]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) fc[2 * c + tt] = row_frag64(ctile + nt * Sub64::ELEMS, 32 * tt, c, lo);
#pragma unroll
    for (int c = 0; c < 4; ++c) fb[c] = tr_frag(btile + nt * Sub64::ELEMS, 16 * c, lo.trp);
  };
  load(0, cc, cb);
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt) {
    if (nt + 1 < N / 32) load(nt + 1, nc, nb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ph = 0; ph < PH; ++ph)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const Frag<bf16> hf = acc_to_frag<bf16>(H[ph][nt], c);
        Y[ph][0] = mma(hf, cc[2 * c], Y[ph][0]);
        Y[ph][1] = mma(hf, cc[2 * c + 1], Y[ph][1]);
      }
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int ph = 0; ph < PH; ++ph) H[ph][nt] = mma(cb[c], xa[ph][c], H[ph][nt]);
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        cc[c] = nc[c];
        cb[c] = nb[c];
      }
    }
  }
}

// ------------------------------------------------------------------ pass 1

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Waves of a workgroup: HG heads of one group, 2 / PH waves per head, each owning PH of the head's two
// 32-column halves (columns 32 (ph0 + ph) .. of x, y and the state).
template <int HG, int PH>
constexpr int lb_waves = HG * (2 / PH);

// Per-wave constants of a workgroup's chunk (both passes).
struct LbWave {
  int w, l, hw, ph0, c0, c1, last, nseg;
  int b, h;           // batch and head of the wave
  float Ah, dtb;
  const bf16* xg;     // x of the wave's head, token 0, column 0
  const bf16* xg0;    // x of the workgroup's first head, token 0, column 0
  const bf16* Bg;     // B of the head's group, token 0
  const bf16* Cg;     // C of the head's group, token 0
  const float* dtg;   // dt of the wave's head, token 0
};
template <int N, int HG, int PH>
__device__ __forceinline__ LbWave lb_wave(const SsdParams& p, int& k, int& b, int& h) {
  const int nhb = p.nheads / HG;
  int chain;
  lb_block(p.nchunks, p.batch * nhb, k, chain);
  b = chain / nhb;
  LbWave c;
  c.w = wave_id();
  c.l = lane_id();
  c.hw = c.w / (2 / PH);
  c.ph0 = PH == 2 ? 0 : (c.w & 1);
  h = (chain - b * nhb) * HG + c.hw;
  const int g = h / (p.nheads / p.ngroups);
  c.c0 = k * p.chunk_len;
  c.c1 = min(p.seqlen, c.c0 + p.chunk_len);
  c.last = p.seqlen - 1;
  c.nseg = (c.c1 - c.c0 + SEG - 1) / SEG;
  c.Ah = p.A[h];
  c.dtb = p.dt_bias ? p.dt_bias[h] : 0.f;
  c.xg = reinterpret_cast<const bf16*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  c.xg0 = c.xg - (int64_t)c.hw * p.x_sh;
  c.Bg = reinterpret_cast<const bf16*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  c.Cg = reinterpret_cast<const bf16*>(p.C) + (int64_t)b * p.C_sb + (int64_t)g * N;
  c.dtg = p.dt + (int64_t)b * p.dt_sb + h;
  c.b = b;
  c.h = h;
  return c;
}

template <int N, int HG>
struct LbStateStage {
  bf16 X[HG][2][Sub64::ELEMS];    // per head: its x tile, two 32-column halves
  bf16 Bt[N / 32][Sub64::ELEMS];  // B tile
  float dt[HG][SEG];              // per head: raw dt
};
// Pass 1 on chunks of at most LB_STATE_SHORT tokens runs two heads per workgroup with two stages (66.5 KB of
// LDS at N = 128), so that two workgroups share a CU and overlap their ramp-up and drain (b2 L4096 H64 N128,
// chunk 512: 21.6 against 22.4 us with four heads and three stages, one workgroup per CU); longer chunks are
// long streams from HBM that prefer the third stage (b1 L131072 H128, chunk 16384: 2% slower with two heads).
constexpr int LB_STATE_SHORT = 1024;
template <int N, int HG>
constexpr int lb_state_nbuf = (HG > 2 && 3 * sizeof(LbStateStage<N, HG>) <= LB_LDS_BYTES) ? 3 : 2;

// Segment si of the chunk into a pass-1 stage: every wave issues exactly N / 8 / NW + 4 PH + 1 loads (its
// share of the B tile, its halves of its head's x tile, its head's dt; rows past the end of the sequence are
// clamped).  part < 0: all of them; else part 0 the B share, part min(1, NT - 1) the x halves and part NT - 1
// the dt (in the same order of issue).
template <int N, int HG, int PH>
__device__ __forceinline__ void lb_state_fetch(const SsdParams& p, const LbWave& c,
                                               LbStateStage<N, HG>* __restrict__ s, int si, int part = -1) {
  constexpr int BB = N / 8 / lb_waves<HG, PH>, NT = N / 32;
  const int pos = c.c0 + si * SEG;
  if (part < 0 || part == 0) fetch_sub64(&s->Bt[0][0], c.Bg, p.B_sl, pos, c.last, c.w * BB, BB);
  if (part < 0 || part == (NT > 1 ? 1 : 0)) fetch_sub64(&s->X[c.hw][0][0], c.xg, p.x_sl, pos, c.last, 4 * c.ph0, 4 * PH);
  if (part < 0 || part == NT - 1) fetch_dt(s->dt[c.hw], c.dtg, p.dt_sl, pos, c.last, lane_id_here());
}

// Segment si of pass 1's reverse walk, its tiles in stage `cur`; segment fsi (if >= 0) is fetched into
// stage `nxt`.  The stage pointers are __restrict__: the compiler otherwise makes every LDS read wait for all
// outstanding global -> LDS loads (it cannot tell that they write another stage).  `more`: the fetch of the
// next segment of the walk is in flight.
template <int N, int HG, int PH, int NBUF>
__device__ __forceinline__ void lb_state_segment(const SsdParams& p, const LbWave& c,
                                                 const LbStateStage<N, HG>* __restrict__ cur,
                                                 LbStateStage<N, HG>* __restrict__ nxt, int si, int fsi, bool more,
                                                 f32x16 (&S)[PH][N / 32], float& R, const DiagMask& dm,
                                                 const LaneOffs& lo) {
  constexpr int LOADS = N / 8 / lb_waves<HG, PH> + 4 * PH + 1;
  if (NBUF == 3 && more) wait_vmem_n<LOADS>();             // this segment's loads; the next one's may fly
  else wait_vmem();
  lds_barrier();                                           // the segment's tiles are in LDS for every wave
  const int pos = c.c0 + si * SEG;
  float dtv;
  const float cs = seg_decay(p, cur->dt[c.hw][c.l], c.dtb, c.Ah, pos + c.l, c.c1, dtv);
  const float cse = readlane_f(cs, SEG - 1);
  // weight of token s relative to the chunk end: exp(R + cse - cs_s) dt_s <= dt_s
  float wb[2];
  halves(__expf(R + cse - cs) * dtv, wb);
  Frag<bf16> xa[PH][4];
  scaled_x<PH>(&cur->X[c.hw][c.ph0][0], wb, dm, lo, xa);
  // segment fsi's loads, issued in parts between the state update's tiles: issued together right after the
  // barrier, every wave's loads queued behind the whole workgroup's at the memory unit (~1K cycles a segment)
  lb_state_update<N, PH>(S, &cur->Bt[0][0], xa, lo, [&](int nt) {
    if (fsi >= 0) lb_state_fetch<N, HG, PH>(p, c, nxt, fsi, nt);
  });
  R += cse;
}

template <int N, int HG, int PH>
__global__ __launch_bounds__(64 * HG * (2 / PH), HG <= 2 ? 2 : 1) void ssd_lb_state_kernel(SsdParams p) {
  constexpr int NT = N / 32;
  constexpr int NBUF = lb_state_nbuf<N, HG>;
  static_assert((N / 8) % lb_waves<HG, PH> == 0, "B tile split evenly over the waves");
  __shared__ LbStateStage<N, HG> st[NBUF];
  int k, b, h;
  const LbWave c = lb_wave<N, HG, PH>(p, k, b, h);
  const int nseg = c.nseg, l = c.l;
  const DiagMask dm = diag_mask(l);
  const LaneOffs lo = lane_offs(l);
  f32x16 S[PH][NT];
#pragma unroll
  for (int ph = 0; ph < PH; ++ph)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) S[ph][nt] = zero16();
  float R = 0.f;                                           // log-decay of the segments after the current one
  // segments are walked last to first: iteration it handles segment nseg - 1 - it, in stage it % NBUF, and
  // fetches segment nseg - it - NBUF into the stage freed by the previous iteration
#pragma unroll
  for (int d = 0; d < NBUF - 1; ++d)
    if (d < nseg) lb_state_fetch<N, HG, PH>(p, c, &st[d], nseg - 1 - d);
  for (int it = 0; it < nseg; it += NBUF) {
#pragma unroll
    for (int u = 0; u < NBUF; ++u)
      if (it + u < nseg) {
        const int si = nseg - 1 - it - u;
        lb_state_segment<N, HG, PH, NBUF>(p, c, &st[u], &st[(u + NBUF - 1) % NBUF], si, si - (NBUF - 1),
                                          it + u + 1 < nseg, S, R, dm, lo);
      }
  }
  // chunk-local state in fragment order (bf16) and the chunk's log-decay
  const int64_t obase = (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
  for (int ph = 0; ph < PH; ++ph)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        bf16x8 v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (bf16)S[ph][nt][8 * q + i];
        *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.chunk_states) + obase + frag_off_bf(nt, c.ph0 + ph, l, q)) = v;
      }
    }
  if (c.ph0 == 0 && l == 0) p.chunk_decay[((int64_t)b * p.nheads + h) * p.nchunks + k] = R;
}

// ------------------------------------------------------------------ pass 2

constexpr int LB_DSEG = 4;   // segments per decay block: their in-segment decays are formed together

// One stage of segment tiles, at most 64 KB: every access is one base register plus a 16-bit immediate.
template <int N, int HG>
struct LbScanStage {
  bf16 Bt[N / 32][Sub64::ELEMS];      // B tile
  bf16 Ct[N / 32][Sub64::ELEMS];      // C tile
  bf16 X[HG][2][Sub64::ELEMS];        // per head: its x tile (two halves)
};
template <int N, int HG, int NW>
struct LbScanSmem {
  LbScanStage<N, HG> st[2];
  Frag<bf16> mt[3][2][64];            // masked (C B^T)^T tiles (s0,t0), (s0,t1), (s1,t1) as B-operand fragments
  float dec[NW][LB_DSEG][2][SEG];     // per wave: [0] cs_t, [1] dt_t of its head, segments of the decay block
  float dcol[HG][HD];                 // D per column of each head
};
// Waves that fetch the segment tiles (the last lb_fetch_waves of the workgroup; the first three compute the
// masked C B^T tiles meanwhile when there are enough waves).
template <int NW>
constexpr int lb_fetch_waves = NW >= 4 ? NW / 2 : NW;

// Masked (C B^T)^T tile ti of the segment: acc[s][t] = C_t . B_s for s <= t, as two B-operand fragments.
template <int N>
__device__ __forceinline__ void cb_tile(int ti, const bf16* btile, const bf16* ctile, Frag<bf16>* out,
                                        const LaneOffs& lo, int l) {
  const int st = (ti == 2) ? 1 : 0, tt = (ti == 0) ? 0 : 1;
  const int half = l >> 5, l32 = l & 31;
  f32x16 acc = zero16();
#pragma unroll
  for (int c = 0; c < N / 16; ++c)
    acc = mma(row_frag64(btile + (c >> 1) * Sub64::ELEMS, 32 * st, c & 1, lo),
              row_frag64(ctile + (c >> 1) * Sub64::ELEMS, 32 * tt, c & 1, lo), acc);
  if (st == tt) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (acc_row(half, r) > l32) acc[r] = 0.f;
  }
  out[l] = acc_to_frag<bf16>(acc, 0);
  out[64 + l] = acc_to_frag<bf16>(acc, 1);
}

// H[ph][nt] += f S on the MFMA unit, for the wave's halves of one state S in bf16 fragment order
// (v[ph][nt][c] = the B-operand fragment of k-step c of tile (nt, ph0 + ph)): A = f I, with f split into bf16
// parts f_hi + f_lo (LO: else f is taken as exact in bf16), so the sum keeps about 16 bits of f.
template <int N, int PH, bool LO>
__device__ __forceinline__ void add_state(f32x16 (&H)[PH][N / 32], const bf16x8 (&v)[PH][N / 32][2], float f,
                                          const DiagMask& dm) {
  Frag<bf16> dh[2], dl[2];
  const float fh = (float)(bf16)f;
  diag_frags(fh, dm, dh);
  if constexpr (LO) diag_frags(f - fh, dm, dl);
#pragma unroll
  for (int ph = 0; ph < PH; ++ph)
#pragma unroll
    for (int nt = 0; nt < N / 32; ++nt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        Frag<bf16> s;
        s.v = v[ph][nt][c];
        H[ph][nt] = mma(dh[c], s, H[ph][nt]);
        if constexpr (LO) H[ph][nt] = mma(dl[c], s, H[ph][nt]);
      }
}

// Segment tiles of pass 2 into one stage, by the fetching waves: each issues exactly lb_fetch_loads loads
// (its share of the B and C tiles and XB of the HG x 8 blocks of the heads' x tiles); the other waves none.
template <int N, int HG, int NW>
struct LbFetch {
  static constexpr int ND = lb_fetch_waves<NW>;
  static constexpr int BB = N / 8 / ND;                    // B (and C) blocks per fetching wave
  static constexpr int XB = HG * 8 / ND;                   // x blocks per fetching wave
  static constexpr int LOADS = 2 * BB + XB;
  static_assert((N / 8) % ND == 0 && (HG * 8) % ND == 0 && (XB % 8 == 0 || 8 % XB == 0), "fetch split");
};
template <int N, int HG, int NW>
__device__ __forceinline__ void lb_scan_fetch(const SsdParams& p, const LbWave& c, LbScanStage<N, HG>* __restrict__ s,
                                              int si) {
  using F = LbFetch<N, HG, NW>;
  const int d = c.w - (NW - F::ND);
  if (d < 0) return;
  const int pos = c.c0 + si * SEG;
  fetch_sub64(&s->Bt[0][0], c.Bg, p.B_sl, pos, c.last, d * F::BB, F::BB);
  fetch_sub64(&s->Ct[0][0], c.Cg, p.C_sl, pos, c.last, d * F::BB, F::BB);
  constexpr int XS = F::XB < 8 ? F::XB : 8;                // blocks per head piece
#pragma unroll
  for (int q = 0; q < F::XB; q += XS) {
    const int gb = d * F::XB + q, hd = gb / 8;
    fetch_sub64(&s->X[hd][0][0], c.xg0 + (int64_t)hd * p.x_sh, p.x_sl, pos, c.last, gb % 8, XS);
  }
}
// Raw dt of the LB_DSEG segments from s0 into the dt slots of the wave's decay block (LB_DSEG loads; tokens
// past the sequence re-read its last one), and their forming in place into cs and dt (tokens past the chunk
// get dt = 0).
__device__ __forceinline__ void lb_dt_fetch(const SsdParams& p, const LbWave& c, float* __restrict__ dec, int s0) {
  const int lane = lane_id_here();
#pragma unroll
  for (int j = 0; j < LB_DSEG; ++j)
    fetch_dt(dec + (2 * j + 1) * SEG, c.dtg, p.dt_sl, min(c.c0 + (s0 + j) * SEG, c.last), c.last, lane);
}
__device__ __forceinline__ void lb_dt_form(const SsdParams& p, const LbWave& c, float* __restrict__ dec, int s0) {
#pragma unroll
  for (int j = 0; j < LB_DSEG; ++j) {
    float dtv;
    const float cs = seg_decay(p, dec[(2 * j + 1) * SEG + c.l], c.dtb, c.Ah, c.c0 + (s0 + j) * SEG + c.l, c.c1, dtv);
    dec[2 * j * SEG + c.l] = cs;
    dec[(2 * j + 1) * SEG + c.l] = dtv;
  }
}

// Segment si of pass 2, its tiles in stage `cur`; stage `nxt` receives segment si + 1.  The stage (and decay block) pointers are __restrict__: the compiler otherwise makes
// every LDS read wait for all outstanding global -> LDS loads (it cannot tell that they write the other stage).
template <int N, int HG, int PH, bool GATE>
__device__ __forceinline__ void lb_scan_segment(const SsdParams& p, const LbWave& c, int si,
                                                LbScanStage<N, HG>* __restrict__ cur,
                                                LbScanStage<N, HG>* __restrict__ nxt, float* __restrict__ dec,
                                                Frag<bf16>* mt, const float* dcol, bf16* yg, const bf16* zg,
                                                f32x16 (&H)[PH][N / 32], float& kappa, const DiagMask& dm,
                                                const LaneOffs& lo) {
  constexpr int NT = N / 32, NW = lb_waves<HG, PH>;
  constexpr int LOADS = LbFetch<N, HG, NW>::LOADS;
  const bf16* bt = &cur->Bt[0][0];
  const bf16* ct = &cur->Ct[0][0];
  const bf16* xw = &cur->X[c.hw][c.ph0][0];
  const int l = c.l, half = l >> 5, l32 = l & 31, nseg = c.nseg;
  const int pos = c.c0 + si * SEG;
  // this segment's tiles: segment 0's here (segment 1's may still fly); a later segment's were waited for
  // before the previous segment's y stores (loads and stores share vmcnt, so a counted wait past stores
  // is not exact)
  if (si == 0) {
    if (nseg > 1) wait_vmem_n<LOADS>();
    else wait_vmem();
  }
  // this head's in-segment decay (lane = token)
  const int dj = si % LB_DSEG;
  const float cs = dec[2 * dj * SEG + l];
  const float dtv = dec[(2 * dj + 1) * SEG + l];
  lds_barrier();                                           // tiles in LDS; the other stage is free
  if (si > 0 && si + 1 < nseg) lb_scan_fetch<N, HG, NW>(p, c, nxt, si + 1);
  if (PH == 1 && p.xsum && pos + l < c.c1) {
    // the sum of x over the wave's 32 channels of token pos + l (the input of h_states), from the x tile (row
    // offsets from a lane index recomputed here: hoisted, they were spilled, and each reload waited for the
    // next segment's tile loads)
    float xs = 0.f;
    const int lh = lane_id_here();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(xw + Sub64::off(lh, 8 * q));
#pragma unroll
      for (int j = 0; j < 8; ++j) xs += (float)v[j];
    }
    p.xsum[(((int64_t)c.b * p.seqlen + pos + lh) * p.nheads + c.h) * 2 + c.ph0] = xs;
  }
  const bool dnext = dj == LB_DSEG - 1 && si + 1 < nseg;  // the next decay block is due
  if (dnext) lb_dt_fetch(p, c, dec, si + 1);
  const float cse = readlane_f(cs, SEG - 1);
  // ---- the segment's three masked C B^T tiles, tile ti by wave ti % NW
  for (int ti = c.w; ti < 3; ti += NW) cb_tile<N>(ti, bt, ct, mt + 128 * ti, lo, l);
  // ---- tokens [a, bnd) per pass: the scale factors e^{-kappa - cs_s} of a pass stay within
  // e^LB_FACT_RANGE, so a segment whose decay range exceeds it takes several passes (a token's own decay,
  // however large, is applied to the state at the start of its pass)
  int a = 0;
  bf16x4 yb[PH][2][4];                                     // the segment's y pieces over the passes
  for (int pass = 0;; ++pass) {
    // the tile reads of a pass stay inside the pass loop (hoisted, the C and B fragments would hold their
    // registers through it): the tile pointers are offset by an opaque zero
    int z0 = 0;
    asm volatile("" : "+s"(z0));
    const bf16* btp = bt + z0;
    const bf16* ctp = ct + z0;
    const bf16* xwp = xw + z0;
    const float csa = readlane_f(cs, a);
    const uint64_t over = __builtin_amdgcn_ballot_w64(l > a && cs < csa - LB_FACT_RANGE);
    const int bnd = over ? (int)__builtin_ctzll(over) : SEG;
    if (-(kappa + readlane_f(cs, bnd - 1)) > LB_FACT_RANGE) {
      const float e = __expf(kappa + csa);               // renormalise: kappa <- -cs_a
#pragma unroll
      for (int ph = 0; ph < PH; ++ph)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) H[ph][nt] *= e;
      kappa = -csa;
    }
    float wb[2], rsb[2];
    halves(l >= a && l < bnd ? __expf(-kappa - cs) * dtv : 0.f, wb);
    halves(__expf(kappa + cs), rsb);
    Frag<bf16> xa[PH][4];
    scaled_x<PH>(xwp, wb, dm, lo, xa);
    f32x16 Y[PH][2];
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) Y[ph][0] = Y[ph][1] = zero16();
    // read-out of the state entering the pass and the state update, fused per state tile
    readout<N, PH>(H, Y, ctp, btp, xa, lo);
    if (pass == 0) lds_barrier();                          // the masked tiles are in LDS
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      Y[ph][0] = mma(xa[ph][0], mt[l], Y[ph][0]);
      Y[ph][0] = mma(xa[ph][1], mt[64 + l], Y[ph][0]);
      Y[ph][1] = mma(xa[ph][0], mt[128 + l], Y[ph][1]);
      Y[ph][1] = mma(xa[ph][1], mt[192 + l], Y[ph][1]);
      Y[ph][1] = mma(xa[ph][2], mt[256 + l], Y[ph][1]);
      Y[ph][1] = mma(xa[ph][3], mt[320 + l], Y[ph][1]);
    }
    // ---- epilogue: y[t][p] = rs_t Y^T[p][t] + D_p x[t][p] for the pass's tokens, in the accumulator layout
    // (lane = token t, 8-byte pieces of 4 columns), kept for the segment's row-chunk stores below (rows past the
    // end of the sequence are computed from clamped rows and not stored)
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      const bf16* xt = xwp + ph * Sub64::ELEMS;
      bf16x4 xv[2][4];
      f32x4 d4[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        d4[q] = *reinterpret_cast<const f32x4*>(dcol + 32 * (c.ph0 + ph) + 8 * q + 4 * half);
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
          xv[tt][q] = *reinterpret_cast<const bf16x4*>(xt + 32 * tt * Sub64::W + lo.piece[q]);
      }
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int t = 32 * tt + l32;
        if (t >= a && t < bnd) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            bf16x4 yo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              float yv = rsb[tt] * Y[ph][tt][4 * q + i] + d4[q][i] * (float)xv[tt][q][i];
              yo[i] = (bf16)yv;
            }
            yb[ph][tt][q] = yo;
          }
        }
      }
    }
    if (bnd >= SEG) break;
    a = bnd;
  }
  {
    // y through the wave's own x sub-tile (no longer read; the same swizzled layout) into 16-byte row chunks:
    // a store instruction then writes 16 rows of 64 contiguous bytes instead of 32 rows of 16, which the
    // memory system drains at about twice the rate.  Before the stores: every load of this wave is complete,
    // in particular the next segment's tiles.
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      bf16* ys = &cur->X[c.hw][c.ph0][0] + ph * Sub64::ELEMS;
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int q = 0; q < 4; ++q) *reinterpret_cast<bf16x4*>(ys + 32 * tt * Sub64::W + lo.piece[q]) = yb[ph][tt][q];
    }
    // the gate y * silu(z) on the same 16-byte row chunks: z is loaded here, so no z registers are held through
    // the segment (the staged y is bf16: the gated value is rounded a second time, within half an ulp more)
    uint4 zc[PH][4];
    if constexpr (GATE) {
#pragma unroll
      for (int ph = 0; ph < PH; ++ph)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = min((l >> 2) + 16 * j, c.c1 - 1 - pos), ch = l & 3;
          zc[ph][j] = *reinterpret_cast<const uint4*>(zg + (int64_t)(pos + r) * p.z_sl + 32 * ph + 8 * ch);
        }
    }
    wait_vmem();
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      const bf16* ys = &cur->X[c.hw][c.ph0][0] + ph * Sub64::ELEMS;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = (l >> 2) + 16 * j, ch = l & 3;
        uint4 v = *reinterpret_cast<const uint4*>(ys + Sub64::off(r, 8 * ch));
        if constexpr (GATE) {
          bf16x8 yv = __builtin_bit_cast(bf16x8, v);
          const bf16x8 zv = __builtin_bit_cast(bf16x8, zc[ph][j]);
#pragma unroll
          for (int i = 0; i < 8; ++i) yv[i] = (bf16)((float)yv[i] * silu_f((float)zv[i]));
          v = __builtin_bit_cast(uint4, yv);
        }
        if (pos + r < c.c1) *reinterpret_cast<uint4*>(yg + (int64_t)(pos + r) * p.y_sl + 32 * ph + 8 * ch) = v;
      }
    }
  }
  kappa += cse;
  if (dnext) lb_dt_form(p, c, dec, si + 1);                // its dt was waited for before the y stores
}

template <int N, int HG, int PH, bool GATE>
__global__ __launch_bounds__(64 * HG * (2 / PH)) void ssd_lb_scan_kernel(SsdParams p) {
  constexpr int NT = N / 32, NW = lb_waves<HG, PH>;
  static_assert((N / 8) % NW == 0, "B and C tiles split evenly over the waves");
  constexpr int LOADS = LbFetch<N, HG, NW>::LOADS;         // loads a fetching wave issues per segment
  constexpr int LB_SLOTS = PH == 1 ? 4 : 3;                // predecessor states in flight in the look-back
  __shared__ LbScanSmem<N, HG, NW> sm;
  int k, b, h;
  const LbWave c = lb_wave<N, HG, PH>(p, k, b, h);
  const int w = c.w, l = c.l, half = l >> 5, l32 = l & 31, nseg = c.nseg, hw = c.hw, ph0 = c.ph0;
  bf16* yg = reinterpret_cast<bf16*>(p.y) + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + 32 * ph0;
  const bf16* zg =
      GATE ? reinterpret_cast<const bf16*>(p.z) + (int64_t)b * p.z_sb + (int64_t)h * p.z_sh + 32 * ph0 : nullptr;
  float* dec = &sm.dec[w][0][0][0];
  sm.dcol[hw][l] = p.D ? (p.D_per_channel ? p.D[h * HD + l] : p.D[h]) : 0.f;
  const DiagMask dm = diag_mask(l);

  // ---- entering state H_k (fp32 accumulators, rows n (state_row_perm order), columns p of each half)
  f32x16 H[PH][NT];
#pragma unroll
  for (int ph = 0; ph < PH; ++ph)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) H[ph][nt] = zero16();
  const int64_t per = (int64_t)HD * N;
  auto load_state = [&](const bf16* s, bf16x8 (&v)[PH][NT][2]) {
#pragma unroll
    for (int ph = 0; ph < PH; ++ph)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          v[ph][nt][q] = *reinterpret_cast<const bf16x8*>(s + frag_off_bf(nt, ph0 + ph, l, q));
  };
  if (p.entering) {
    // entering states precomputed by ssd_state_pass_kernel (bf16, fragment order)
    bf16x8 v[PH][NT][2];
    load_state(reinterpret_cast<const bf16*>(p.entering) + (((int64_t)b * p.nchunks + k) * p.nheads + h) * per, v);
    lb_dt_fetch(p, c, dec, 0);
    lb_scan_fetch<N, HG, NW>(p, c, &sm.st[0], 0);
    add_state<N, PH, false>(H, v, 1.f, dm);
  } else {
    // look-back: lane i < k holds T_i; f_j = exp(T_{j+1} + .. + T_{k-1}) = exp(P_{k-1} - P_j), and the initial
    // state enters with exp(P_{k-1}).  LB_SLOTS predecessor states are in flight at a time (indices past
    // k - 1 re-read state k - 1 and are not summed).
    const float* T = p.chunk_decay + ((int64_t)b * p.nheads + h) * p.nchunks;
    const bf16* sbase = reinterpret_cast<const bf16*>(p.chunk_states) + ((int64_t)b * p.nchunks * p.nheads + h) * per;
    const int64_t cstride = (int64_t)p.nheads * per;       // elements between consecutive chunks
    const float tl = l < k ? T[l] : 0.f;
    bf16x8 v[LB_SLOTS][PH][NT][2];
    if (k > 0) {
#pragma unroll
      for (int u = 0; u < LB_SLOTS; ++u) load_state(sbase + min(u, k - 1) * cstride, v[u]);
    }
    lb_dt_fetch(p, c, dec, 0);
    lb_scan_fetch<N, HG, NW>(p, c, &sm.st[0], 0);
    const float Pi = wave_incl_scan(tl);
    const float Ptot = readlane_f(Pi, 63);
    const float f = __expf(Ptot - Pi);
    if (p.init_state) {
      const float e0 = __expf(Ptot);
#pragma unroll
      for (int ph = 0; ph < PH; ++ph) {
        const float* h0 = p.init_state + ((int64_t)b * p.nheads + h) * per + (int64_t)(32 * (ph0 + ph) + l32) * N;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const f32x4 hv = *reinterpret_cast<const f32x4*>(h0 + 32 * nt + state_row_perm(8 * q + 4 * half));
#pragma unroll
            for (int i = 0; i < 4; ++i) H[ph][nt][4 * q + i] = e0 * hv[i];
          }
      }
    }
    for (int j = 0; j < k; j += LB_SLOTS) {
#pragma unroll
      for (int u = 0; u < LB_SLOTS; ++u)
        if (j + u < k) {
          add_state<N, PH, true>(H, v[u], readlane_f(f, j + u), dm);
          if (j + u + LB_SLOTS < k) load_state(sbase + (j + u + LB_SLOTS) * cstride, v[u]);
        }
    }
  }
  // the first decay block: a fetching wave lets its segment-0 tile loads fly, the others have none in flight
  if (w >= NW - LbFetch<N, HG, NW>::ND) wait_vmem_n<LOADS>();
  else wait_vmem();
  lb_dt_form(p, c, dec, 0);
  if (nseg > 1) lb_scan_fetch<N, HG, NW>(p, c, &sm.st[1], 1);

  const LaneOffs lo = lane_offs(l);
  float kappa = 0.f;                                       // H_true = e^kappa H
  for (int si = 0; si < nseg; ++si) {
    const int cur = si & 1;
    lb_scan_segment<N, HG, PH, GATE>(p, c, si, &sm.st[cur], &sm.st[cur ^ 1], dec, &sm.mt[0][0][0], sm.dcol[hw],
                                     yg, zg, H, kappa, dm, lo);
  }
  // final state (last chunk): H_true = e^kappa H, canonical (b, H, P, N) fp32
  if (p.final_state && k == p.nchunks - 1) {
    const float e = __expf(kappa);
#pragma unroll
    for (int ph = 0; ph < PH; ++ph) {
      float* fo = p.final_state + ((int64_t)b * p.nheads + h) * per + (int64_t)(32 * (ph0 + ph) + l32) * N;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          f32x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = e * H[ph][nt][4 * q + i];
          *reinterpret_cast<f32x4*>(fo + 32 * nt + state_row_perm(8 * q + 4 * half)) = v;
        }
    }
  }
}

constexpr int LB_PH = 1;   // halves per wave of the two-pass prefill (1: two waves per head)

template <int N, int HG>
hipError_t launch_lb_t(const SsdParams& p, hipStream_t stream) {
  constexpr int NW = lb_waves<HG, LB_PH>;
  dim3 grid((unsigned)(p.nchunks * p.batch * (p.nheads / HG)));
  constexpr int HS = HG < 2 ? HG : 2;                      // pass 1's heads per workgroup on short chunks
  if (p.chunk_len <= LB_STATE_SHORT)
    hipLaunchKernelGGL((ssd_lb_state_kernel<N, HS, LB_PH>), dim3((unsigned)(p.nchunks * p.batch * (p.nheads / HS))),
                       dim3(64 * lb_waves<HS, LB_PH>), 0, stream, p);
  else
    hipLaunchKernelGGL((ssd_lb_state_kernel<N, HG, LB_PH>), grid, dim3(64 * NW), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.entering) {
    SsdParams q = p;
    q.final_state = nullptr;                               // the scan writes the final state
    q.state_perm = 1;                                      // the chunk states' rows are in state_row_perm order
    e = launch_ssd_state_pass(q, stream);
    if (e != hipSuccess) return e;
  }
  if (p.z) hipLaunchKernelGGL((ssd_lb_scan_kernel<N, HG, LB_PH, true>), grid, dim3(64 * NW), 0, stream, p);
  else hipLaunchKernelGGL((ssd_lb_scan_kernel<N, HG, LB_PH, false>), grid, dim3(64 * NW), 0, stream, p);
  return hipGetLastError();
}

template <int N>
hipError_t launch_lb_n(const SsdParams& p, hipStream_t stream) {
  switch (p.heads_per_wg) {
    case 4: return launch_lb_t<N, 4>(p, stream);
    case 2: return launch_lb_t<N, 2>(p, stream);
    case 1: return launch_lb_t<N, 1>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool ssd_lb_supported(int dtype, int dstate) { return dtype == DT_BF16 && (dstate == 64 || dstate == 128); }

hipError_t launch_ssd_lb(const SsdParams& p, hipStream_t stream) {
  if (p.dstate == 128) return launch_lb_n<128>(p, stream);
  if (p.dstate == 64) return launch_lb_n<64>(p, stream);
  return hipErrorInvalidValue;
}

}  // namespace mh
