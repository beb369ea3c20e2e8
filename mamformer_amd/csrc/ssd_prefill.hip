// Mamba-2 SSD chunked-scan prefill for gfx950.
//
// Recurrence (per batch b, head h with group g = h / (H/G), channel p, state n):
//     h_t = exp(A_h dt_t) h_{t-1} + dt_t x_t[p] B_t[g, n]
//     y_t[p] = sum_n C_t[g, n] h_t[p, n] + D x_t[p]
// i.e. the reference's selective_scan (mamformer/layers/mamba2.py:84-126) in the
// per-head SSD parameterisation, with an optional initial state (prefill of a
// cached sequence) and the final state returned for the decode cache.
//
// Decomposition (four launches on the caller's stream):
//   0. ssd_seg_frags    grid (nseg, G, b): per 64-token segment of each group, the
//      MFMA operand fragments every head of the group shares -- B^T (n x token)
//      and the causally masked (C B^T)^T tile -- written once to the workspace.
//   1. ssd_chunk_state  grid (nchunks, H/HG, b): the chunk-local final state
//          S_k[p, n] = sum_{s in k} exp(sum_{s<tau in k} A dt_tau) dt_s x_s[p] B_s[n]
//      and the chunk's total log-decay T_k, walking the chunk in 64-token segments
//      with S in MFMA accumulators.
//   2. ssd_state_pass   elementwise over (b, h, P*N): H_0 = h0, H_{k+1} = e^{T_k} H_k + S_k.
//      Writes the *entering* state H_k over S_k and the final state.
//   3. ssd_chunk_scan   grid (nchunks, H/HG, b): walks the chunk in 64-token
//      segments with the running state in MFMA accumulators.  With cs_t the
//      in-segment inclusive cumulative log-decay (cs_t <= 0, non-increasing):
//          y_t  = e^{cs_t} C_t H^T + sum_{s<=t} e^{cs_t - cs_s} (C_t . B_s) dt_s x_s + D x_t
//          H   <- e^{cs_end} H + sum_s e^{cs_end - cs_s} dt_s x_s B_s^T
//      The state is carried lazily as H_true = e^kappa H, so a segment needs one
//      scaled operand xs_s = e^{-kappa - cs_s} dt_s x_s for both terms:
//          y_t = e^{kappa + cs_t} (C_t H^T + sum_{s<=t} M[t][s] xs_s),  H += B^T xs,  kappa += cs_end
//      and H is rescaled only when a factor would pass e^{FACT_RANGE}.  A segment
//      whose own decay range exceeds FACT_RANGE takes an exact path with the
//      per-element factor e^{cs_t - cs_s} (wave-uniform branch).
// Work split: a workgroup owns HG heads of one group with two waves per head;
// wave w handles head w / 2 and the 32 state columns p of half w % 2, so each
// wave's state is N/32 accumulator tiles.  Transposes needed by the
// token-contracted MFMAs (B^T, x^T) are done on the MFMA unit itself: a
// row-loaded tile times an identity fragment lands in the accumulator layout
// that the next MFMA consumes.
// Memory: every segment's inputs (shared fragments, C tile, x tile, dt) are
// fetched straight into LDS (global_load_lds, no register staging) one or two
// segments ahead of their use, and waited for with vmcnt only where consumed;
// barriers inside the loops order LDS traffic only (no memory fence, which
// would also wait for the prefetch).  Each wave owns the 32-column half of its
// head's x tile, so it stages its y columns in place of x and writes them to
// HBM one segment later.  LDS tiles are XOR-swizzled per row for
// conflict-free fragment reads; the chunk-state workspace is kept in MFMA
// fragment order (frag_off / frag_off_bf).
// bf16 I/O uses 32x32x16 bf16 MFMAs, fp32 I/O 32x32x2 fp32 MFMAs; accumulation is fp32.
#include "common.h"
#include "launch.h"
#include "ssd_shared.h"
#include "tiles.h"

namespace mh {

constexpr float FACT_RANGE = 60.f;   // max exponent of an operand scale factor

// ------------------------------------------------------------------ helpers

// x^T of a wave's x half tile (lane = p, tokens on the k axis, KSET order) as
// 4 fragments, each token scaled by sa[token].
template <typename TM, typename T>
__device__ __forceinline__ void xt_frags(const T* xtile, const float* sa, const Frag<TM> (&id)[2], int half, int l32,
                                         Frag<TM> (&xa)[4]) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    f32x16 xt = zero16();
#pragma unroll
    for (int c = 0; c < 2; ++c) xt = mma(xrow_frag<TM, T>(xtile, 32 * st + l32, 16 * c + 8 * half), id[c], xt);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float s[8];
      kset_vals(sa, 2 * st + c, half, s);
#pragma unroll
      for (int j = 0; j < 8; ++j) xa[2 * st + c].set(j, xt[8 * c + j] * s[j]);
    }
  }
}

// Operand fragments one segment of a group shares among all its heads, in the
// layout written by ssd_seg_frags and copied verbatim (1 KB blocks) into LDS:
//   bt[nt][c][lane]  B^T A-operand fragment (row n = 32 nt + lane % 32, k = token 16 c + KSET)
//   cb[ti][c][lane]  masked (C B^T)^T tile ti in {(s 0, t 0), (s 0, t 1), (s 1, t 1)} as a
//                    B-operand fragment (column t, k = token s 16 c + KSET within the s-tile)
//   ct[nt][c][tt][lane]  C^T as a B-operand fragment (column t = 32 tt + lane % 32,
//                    k = state n = 32 nt + 16 c + KSET) for the state read-out
template <typename TM, int N>
struct SegFrags {
  Frag<TM> bt[N / 32][4][64];
  Frag<TM> cb[3][2][64];
  Frag<TM> ct[N / 32][2][2][64];
};
template <typename TM, int N>
constexpr int frag_blocks = (int)(sizeof(SegFrags<TM, N>) / 1024);
template <typename TM, int N>
constexpr int bt_blocks = (int)(sizeof(Frag<TM>) * (N / 32) * 4 * 64 / 1024);
static_assert(sizeof(SegFrags<bf16, 128>) % 1024 == 0 && sizeof(SegFrags<float, 64>) % 1024 == 0, "1 KB blocks");

// Per-stage tiles.
template <typename T, typename TM, int N, int HG>
struct ScanStage {
  SegFrags<TM, N> fr;
  T X[2 * HG][SEG * 32];      // per wave: its half of its head's x tile (y staged in place)
  float dt[2 * HG][SEG];      // per wave: raw dt of its head for the segment's tokens
};
template <typename T, typename TM, int N, int HG>
struct StateStage {
  Frag<TM> bt[N / 32][4][64];
  T X[2 * HG][SEG * 32];
  float dt[2 * HG][SEG];
};

template <typename T, typename TM, int N, int HG, int NBUF>
struct ScanSmem {
  ScanStage<T, TM, N, HG> st[NBUF];
  float sa[2 * HG][SEG];      // per wave: per-token operand scale
  float cs[2 * HG][SEG];      // per wave: in-segment cumulative log-decay
  float dcol[HG][HD];         // D per column of each head
};
template <typename T, typename TM, int N, int HG, int NBUF>
struct StateSmem {
  StateStage<T, TM, N, HG> st[NBUF];
  float sb[2 * HG][SEG];
};

// Tiles are fetched ahead into as many stages as fit in the 160 KB of LDS.
constexpr size_t LDS_BYTES = 160 * 1024;
template <typename T, typename TM, int N, int HG>
constexpr int scan_nbuf = sizeof(ScanSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1;
template <typename T, typename TM, int N, int HG>
constexpr int state_nbuf = sizeof(StateSmem<T, TM, N, HG, 3>) <= LDS_BYTES ? 3
                           : (sizeof(StateSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1);

// State read-out of one wave: Y^T[p][t] += sum_n H[p][n] C^T[n][t] for the two 32-token t-tiles of the
// segment (H as A operand straight from the accumulators, converted once for both; C^T fragments
// precomputed per segment).
template <typename TM, int N>
__device__ __forceinline__ void readout(const f32x16 (&H)[N / 32], const Frag<TM> (&ct)[N / 32][2][2][64], int l,
                                        f32x16& Y0, f32x16& Y1) {
  // C^T fragments of state tile nt + 1 are read from LDS while the MFMAs of tile nt run
  Frag<TM> cur[2][2], nxt[2][2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) cur[c][tt] = ct[0][c][tt][l];
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt) {
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) nxt[c][tt] = ct[nt + 1][c][tt][l];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const Frag<TM> hf = acc_to_frag<TM>(H[nt], c);
      Y0 = mma(hf, cur[c][0], Y0);
      Y1 = mma(hf, cur[c][1], Y1);
    }
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) cur[c][tt] = nxt[c][tt];
    }
  }
}

// H[n][p] += sum_s B^T[n][s] xf[s][p] over the segment's 64 tokens.
template <typename TM, int N>
__device__ __forceinline__ void state_update(f32x16 (&H)[N / 32], const Frag<TM> (&bt)[N / 32][4][64],
                                             const Frag<TM> (&xf)[4], int l) {
  // B^T fragments of state tile nt + 1 are read from LDS while the MFMAs of tile nt run
  Frag<TM> cur[4], nxt[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) cur[c] = bt[0][c][l];
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt) {
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) nxt[c] = bt[nt + 1][c][l];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < 4; ++c) H[nt] = mma(cur[c], xf[c], H[nt]);
    if (nt + 1 < N / 32) {
#pragma unroll
      for (int c = 0; c < 4; ++c) cur[c] = nxt[c];
    }
  }
}

// Workspace layout: [chunk states][chunk log-decays][segment fragments], each 256-byte aligned.
// ------------------------------------------------------------------ kernel 0

// One workgroup of 8 waves per (segment, group, batch): 3 + 2 N/32 work items
// (the C B^T tiles and the B^T blocks), wave w taking items w and w + 8, then
// the C^T fragments, read straight out of the C tile.
template <typename T, typename TM, int N>
__global__ __launch_bounds__(512) void ssd_seg_frags_kernel(SsdParams p) {
  using TB = Tile<T, N>;
  static_assert(TB::NBLK % 8 == 0, "B and C tiles split evenly over 8 waves");
  __shared__ T Bs[SEG * N];
  __shared__ T Cs[SEG * N];
  const int sgi = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tok0 = sgi * SEG;
  const int len = min(SEG, p.seqlen - tok0);
  const int last = p.seqlen - 1;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const T* Cg = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + (int64_t)g * N;
  constexpr int BPW = TB::NBLK / 8;
  fetch_tile<T, N>(Bs, Bg, p.B_sl, tok0, last, w * BPW, BPW, l);
  fetch_tile<T, N>(Cs, Cg, p.C_sl, tok0, last, w * BPW, BPW, l);
  wait_vmem();
  lds_barrier();
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);
  auto* out = reinterpret_cast<SegFrags<TM, N>*>(p.seg_frags) + ((int64_t)b * p.ngroups + g) * p.nseg + sgi;
  constexpr int NBT = 2 * (N / 32);
  for (int it = w; it < 3 + NBT; it += 8) {
    if (it < 3) {
      const int st = (it == 2) ? 1 : 0, tt = (it == 0) ? 0 : 1;
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < N / 16; ++c)
        acc = mma(row_frag<TM, T, N>(Bs, 32 * st + l32, 16 * c + 8 * half),
                  row_frag<TM, T, N>(Cs, 32 * tt + l32, 16 * c + 8 * half), acc);
      const int tl = 32 * tt + l32;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s = 32 * st + acc_row(half, r);
        if (!(s <= tl && s < len)) acc[r] = 0.f;
      }
      out->cb[it][0][l] = acc_to_frag<TM>(acc, 0);
      out->cb[it][1][l] = acc_to_frag<TM>(acc, 1);
    } else {
      const int blk = it - 3;
      const f32x16 acc = mfma_transpose<TM, T, N>(Bs, 32 * (blk & 1), 32 * (blk >> 1), id, half, l32);
      out->bt[blk >> 1][2 * (blk & 1)][l] = acc_to_frag<TM>(acc, 0);
      out->bt[blk >> 1][2 * (blk & 1) + 1][l] = acc_to_frag<TM>(acc, 1);
    }
  }
  // C^T read-out fragments: (nt, c, tt) = f, two per wave
  for (int f = w; f < (N / 32) * 4; f += 8) {
    const int nt = f >> 2, c = (f >> 1) & 1, tt = f & 1;
    out->ct[nt][c][tt][l] = kset_frag<TM, T, N>(Cs, 32 * tt + l32, 32 * nt + 16 * c, half);
  }
}

// ------------------------------------------------------------------ kernel 1

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(128 * HG) void ssd_chunk_state_kernel(SsdParams p) {
  constexpr int NBUF = state_nbuf<T, TM, N, HG>;
  constexpr int DIST = NBUF - 1;                           // segments fetched ahead (0: fetch-then-wait)
  using SM = StateSmem<T, TM, N, HG, NBUF>;
  __shared__ SM sm;
  constexpr int NT = N / 32, NW = 2 * HG;
  using TX = XHalf<T>;
  constexpr int FB = bt_blocks<TM, N>;
  static_assert(FB % NW == 0, "every wave fetches the same number of fragment blocks");
  constexpr int BPW = FB / NW;
  constexpr int LOADS = BPW + TX::NBLK + 1;                // loads one wave issues per segment
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int j = w >> 1, ph = w & 1;
  const int h = blockIdx.y * HG + j;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const int last = p.seqlen - 1;
  const float Ah = p.A[h];
  const float dtb = p.dt_bias ? p.dt_bias[h] : 0.f;
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh + 32 * ph;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  const char* fg = reinterpret_cast<const char*>(reinterpret_cast<const SegFrags<TM, N>*>(p.seg_frags) +
                                                 ((int64_t)b * p.ngroups + g) * p.nseg + c0 / SEG);
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);

  // S_true = e^kappa * S (kappa <= 0 carried lazily; S is rescaled only when a factor would
  // pass e^{FACT_RANGE}), so a segment adds B^T (e^{-kappa - cs_s} dt_s x_s) without touching S.
  f32x16 S[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) S[nt] = zero16();
  float kappa = 0.f, total = 0.f;

  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  // every wave issues exactly LOADS loads per segment (rows past the end are clamped), so vmcnt counts them
  // (issued in two parts so the x half can be spread into the compute of the current segment)
  auto fetch_a = [&](int seg) {
    auto& sg = sm.st[seg % NBUF];
    fetch_blocks(reinterpret_cast<char*>(sg.bt), fg + (size_t)seg * sizeof(SegFrags<TM, N>), w * BPW, BPW, l);
    fetch_dt(sg.dt[w], dtg, p.dt_sl, c0 + seg * SEG, last, l);
  };
  auto fetch_b = [&](int seg) { fetch_xhalf<T>(sm.st[seg % NBUF].X[w], xg, p.x_sl, c0 + seg * SEG, last, l); };
  auto fetch = [&](int seg) { fetch_a(seg); fetch_b(seg); };
#pragma unroll
  for (int d = 0; d < (DIST > 0 ? DIST : 1); ++d)          // segments 0 .. DIST-1 in flight before the loop
    if (d < nseg) fetch(d);

  for (int si = 0; si < nseg; ++si) {
    // lane-dependent LDS addresses are recomputed each segment instead of hoisted (and spilled)
    int lq = l;
    asm volatile("" : "+v"(lq));
    const int ll = lq, halfq = lq >> 5, l32q = lq & 31;
    const int pos = c0 + si * SEG;
    auto& sg = sm.st[si % NBUF];
    if constexpr (DIST == 0) {
      if (si > 0) {
        lds_barrier();                                     // every wave is done with the previous tiles
        fetch(si);
      }
    }
    if (DIST == 2 && si + 1 < nseg) wait_vmem_n<LOADS>();  // this segment's loads; the next one's may fly
    else wait_vmem();
    lds_barrier();                                         // this segment's tiles are in LDS
    if constexpr (DIST > 0) {
      if (si + DIST < nseg) fetch_a(si + DIST);
    }
    float dtv;
    const float cs = seg_decay(p, sg.dt[w][ll], dtb, Ah, pos + l, c1, dtv);
    const float cse = lane_val(cs, 63);
    float wsc;                                             // per-token operand scale (wave-uniform choice)
    if (-cse > FACT_RANGE) {                               // very strong decay: carry S exactly through it
      const float e = __expf(kappa + cse);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) S[nt] *= e;
      kappa = 0.f;
      wsc = __expf(cse - cs);
    } else {
      if (-(kappa + cse) > FACT_RANGE) {                   // renormalise: S_true = e^kappa S
        const float e = __expf(kappa);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) S[nt] *= e;
        kappa = 0.f;
      }
      wsc = __expf(-kappa - cs);
      kappa += cse;
    }
    sm.sb[w][ll] = wsc * dtv;                              // wave-private: read back by this wave only
    Frag<TM> xw[4];
    xt_frags<TM, T>(sg.X[w], sm.sb[w], id, halfq, l32q, xw);
    if constexpr (DIST > 0) {
      if (si + DIST < nseg) fetch_b(si + DIST);
    }
    state_update<TM, N>(S, sg.bt, xw, ll);
    total += cse;
  }
  {
    const float e = __expf(kappa);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) S[nt] *= e;
  }

  // chunk-local state in fragment order: bf16 for bf16 I/O (the scan consumes the entering state as bf16
  // MFMA operands anyway), fp32 otherwise
  const int64_t obase = (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        bf16x8 v;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (bf16)S[nt][8 * q + i];
        *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.chunk_states) + obase + frag_off_bf(nt, ph, l, q)) = v;
      }
    } else {
      f32x4* o4 = reinterpret_cast<f32x4*>(p.chunk_states + obase + frag_off(nt, ph, l));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f32x4 v;
        v[0] = S[nt][4 * q]; v[1] = S[nt][4 * q + 1]; v[2] = S[nt][4 * q + 2]; v[3] = S[nt][4 * q + 3];
        o4[q] = v;
      }
    }
  }
  if (l == 0 && ph == 0) p.chunk_decay[((int64_t)b * p.nheads + h) * p.nchunks + k] = total;
}

// ------------------------------------------------------------------ kernel 2

// Entering states for the scan kernel: fp32 in place of fp32 S_k, or (bf16 I/O, where the chunk states
// are bf16 and the scan consumes the state as bf16 MFMA operands) bf16 in a separate array of the same
// fragment order.  The running sum and the final state are fp32.
template <typename TE>
__global__ __launch_bounds__(256) void ssd_state_pass_kernel(SsdParams p) {
  // 8 consecutive workspace elements per thread (16-byte bf16 accesses); the chunk states of up to KB chunks are
  // loaded before any entering state is stored, so the loads are not ordered behind the stores.
  constexpr int KB = 8;
  const int bh = blockIdx.y;
  const int b = bh / p.nheads, h = bh - b * p.nheads;
  const int per = HD * p.dstate;                  // state elements per (b, h)
  const int e8 = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (e8 >= per) return;
  const bool bfs = sizeof(TE) == 2;               // bf16 states in the frag_off_bf order
  const int ci0 = canon_index(e8, p.dstate, p.state_perm, bfs);   // two runs of 4 canonical n
  const int ci1 = canon_index(e8 + 4, p.dstate, p.state_perm, bfs);
  f32x4 H[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) H[u][0] = H[u][1] = H[u][2] = H[u][3] = 0.f;
  if (p.init_state) {
    H[0] = *reinterpret_cast<const f32x4*>(p.init_state + (int64_t)bh * per + ci0);
    H[1] = *reinterpret_cast<const f32x4*>(p.init_state + (int64_t)bh * per + ci1);
  }
  const float* dec = p.chunk_decay + (int64_t)bh * p.nchunks;
  for (int k0 = 0; k0 < p.nchunks; k0 += KB) {
    f32x4 S[KB][2];
    float a[KB];
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (k0 + j < p.nchunks) {
        const int64_t idx = (((int64_t)b * p.nchunks + k0 + j) * p.nheads + h) * per + e8;
        if constexpr (sizeof(TE) == 4) {
          S[j][0] = *reinterpret_cast<const f32x4*>(p.chunk_states + idx);
          S[j][1] = *reinterpret_cast<const f32x4*>(p.chunk_states + idx + 4);
        } else {
          const bf16x8 sb = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.chunk_states) + idx);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            S[j][0][i] = (float)sb[i];
            S[j][1][i] = (float)sb[4 + i];
          }
        }
        a[j] = dec[k0 + j];
      }
    }
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      if (k0 + j < p.nchunks) {
        const int64_t idx = (((int64_t)b * p.nchunks + k0 + j) * p.nheads + h) * per + e8;
        if constexpr (sizeof(TE) == 4) {
          *reinterpret_cast<f32x4*>(p.chunk_states + idx) = H[0];
          *reinterpret_cast<f32x4*>(p.chunk_states + idx + 4) = H[1];
        } else {
          bf16x8 hb;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hb[i] = (bf16)H[0][i];
            hb[4 + i] = (bf16)H[1][i];
          }
          *reinterpret_cast<bf16x8*>(reinterpret_cast<bf16*>(p.entering) + idx) = hb;
        }
        const float d = __expf(a[j]);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
          for (int i = 0; i < 4; ++i) H[u][i] = d * H[u][i] + S[j][u][i];
      }
    }
  }
  if (p.final_state) {
    *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * per + ci0) = H[0];
    *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * per + ci1) = H[1];
  }
}

// ------------------------------------------------------------------ kernel 3

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(128 * HG) void ssd_chunk_scan_kernel(SsdParams p) {
  constexpr int NBUF = scan_nbuf<T, TM, N, HG>;
  using SM = ScanSmem<T, TM, N, HG, NBUF>;
  using Stage = ScanStage<T, TM, N, HG>;
  constexpr int NT = N / 32, NW = 2 * HG;
  using TX = XHalf<T>;
  constexpr int FB = frag_blocks<TM, N>;
  constexpr int FPW = (FB + NW - 1) / NW;                  // fragment blocks fetched per wave (the last ones fewer)
  __shared__ SM sm;
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int j = w >> 1, ph = w & 1;                       // head of the workgroup, 32-column half of P
  const int h = blockIdx.y * HG + j;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const int last = p.seqlen - 1;
  const float Ah = p.A[h];
  const float dtb = p.dt_bias ? p.dt_bias[h] : 0.f;
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh + 32 * ph;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  const char* fg = reinterpret_cast<const char*>(reinterpret_cast<const SegFrags<TM, N>*>(p.seg_frags) +
                                                 ((int64_t)b * p.ngroups + g) * p.nseg + c0 / SEG);
  T* yg = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + 32 * ph;
  // optional output gate y <- y * silu(z): the z rows of a segment are loaded one segment before its y is
  // stored (bf16: into registers right after the tiles barrier; fp32: at the store)
  const T* zg = p.z ? reinterpret_cast<const T*>(p.z) + (int64_t)b * p.z_sb + (int64_t)h * p.z_sh + 32 * ph
                    : nullptr;
  constexpr bool ZPRE = sizeof(T) == 2;
  uint4 zv[TX::NBLK];
  const int f0 = w * FPW, fn = max(0, min(FPW, FB - f0));
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);
  if (ph == 0) sm.dcol[j][l] = p.D ? (p.D_per_channel ? p.D[h * HD + l] : p.D[h]) : 0.f;

  // Entering state H_k (fragment-native workspace order), columns of this wave's P-half.
  f32x16 H[NT];
  {
    const int64_t hidx = (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const bf16x8 v = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p.entering) + hidx +
                                                             frag_off_bf(nt, ph, l, q));
#pragma unroll
          for (int i = 0; i < 8; ++i) H[nt][8 * q + i] = (float)v[i];
        }
      } else {
        const f32x4* h4 = reinterpret_cast<const f32x4*>(p.chunk_states + hidx + frag_off(nt, ph, l));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 v = h4[q];
          H[nt][4 * q] = v[0]; H[nt][4 * q + 1] = v[1]; H[nt][4 * q + 2] = v[2]; H[nt][4 * q + 3] = v[3];
        }
      }
    }
  }
  float kappa = 0.f;
  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  // a segment's fetch: the tiles all heads share, and this wave's x half and dt
  auto fetch_shared = [&](int seg, Stage& sg) {
    fetch_blocks(reinterpret_cast<char*>(&sg.fr), fg + (size_t)seg * sizeof(SegFrags<TM, N>), f0, fn, l);
  };
  auto fetch_own = [&](int seg, Stage& sg) {
    const int pos = c0 + seg * SEG;
    fetch_xhalf<T>(sg.X[w], xg, p.x_sl, pos, last, l);
    fetch_dt(sg.dt[w], dtg, p.dt_sl, pos, last, l);
  };
  fetch_shared(0, sm.st[0]);
  fetch_own(0, sm.st[0]);

  for (int si = 0; si < nseg; ++si) {
    // lane-dependent LDS addresses are recomputed each segment instead of hoisted (and spilled)
    int lq = l;
    asm volatile("" : "+v"(lq));
    const int ll = lq, halfq = lq >> 5, l32q = lq & 31;
    const int pos = c0 + si * SEG;
    const int cur = (NBUF == 2) ? (si & 1) : 0;
    auto& sg = sm.st[cur];
    T* xt = sg.X[w];
    if constexpr (NBUF == 1) {
      if (si > 0) {
        if (zg && !ZPRE) load_zhalf<T>(zg + (int64_t)(pos - SEG) * p.z_sl, p.z_sl, SEG - 1, ll, zv);
        store_yhalf<T>(yg + (int64_t)(pos - SEG) * p.y_sl, p.y_sl, xt, SEG, ll,   // y of the previous segment
                       zg != nullptr, zv);
        lds_barrier();                                     // every wave is done with the previous tiles
        fetch_shared(si, sg);
        fetch_own(si, sg);
      }
    }
    auto& og = sm.st[cur ^ 1];
    uint4 yv[TX::NBLK];
    if constexpr (NBUF == 2) {
      wait_vmem();                                         // this segment's tiles (and the last y stores)
      // y of the previous segment (a full one: only a chunk's last segment is partial), staged by this wave in
      // place of its x in the other stage: read out before that stage is refilled, with no fetch in flight (an
      // LDS read behind a pending direct-to-LDS load would wait for it).
      if (si > 0) {
        if (zg && !ZPRE) load_zhalf<T>(zg + (int64_t)(pos - SEG) * p.z_sl, p.z_sl, SEG - 1, ll, zv);
        load_yhalf<T>(og.X[w], ll, yv);
        if (zg) gate_chunks<T>(yv, zv);
        store_yhalf_full<T>(yg + (int64_t)(pos - SEG) * p.y_sl, p.y_sl, yv, ll);
      }
      lds_barrier();                                       // this segment's tiles are in LDS; the other stage is free
      if (si + 1 < nseg) fetch_shared(si + 1, og);
    } else {
      wait_vmem();
      lds_barrier();                                       // this segment's tiles are in LDS
    }
    if (ZPRE && zg) load_zhalf<T>(zg + (int64_t)pos * p.z_sl, p.z_sl, c1 - 1 - pos, ll, zv);   // for its y store

    // ---- this head's in-segment decay (lane = token).  H_true = e^kappa H (kappa <= 0 carried lazily).
    float dtv;
    const float cs = seg_decay(p, sg.dt[w][ll], dtb, Ah, pos + l, c1, dtv);
    const float cse = lane_val(cs, 63);
    const bool fact = (-cse <= FACT_RANGE);               // wave-uniform
    if (!fact || -(kappa + cse) > FACT_RANGE) {
      const float e = __expf(kappa);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) H[nt] *= e;
      kappa = 0.f;
    }
    sm.sa[w][ll] = (fact ? __expf(-kappa - cs) : 1.f) * dtv;   // wave-private scratch
    sm.cs[w][ll] = cs;

    // ---- per wave: head j, p-tile ph.  Y^T[p][t] = sum_n H[p][n] C^T[n][t] + sum_s xa^T[p][s] M^T[s][t]
    Frag<TM> xa[4];
    xt_frags<TM, T>(xt, sm.sa[w], id, halfq, l32q, xa);
    if constexpr (NBUF == 2) {
      if (si + 1 < nseg) fetch_own(si + 1, og);          // the next segment's own tiles, issued apart from the rest
    }
    const float cs0 = sm.cs[w][l32q], cs1 = sm.cs[w][32 + l32q];
    f32x16 Y0 = zero16(), Y1 = zero16();
    // y[t][p] = rs_t Y + D x, staged in place of x
    auto epilogue = [&](float rs0, float rs1) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int tl = 32 * tt + l32q;
        const float rsc = tt ? rs1 : rs0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int p0 = 8 * q + 4 * halfq;                // 4 consecutive columns of the half, inside one chunk
          T* xp = xt + TX::chunk(tl, (unsigned)p0 / TX::EPC) + ((unsigned)p0 % TX::EPC);
          const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.dcol[j][32 * ph + p0]);
          if constexpr (sizeof(T) == 2) {
            const bf16x4 xv = *reinterpret_cast<const bf16x4*>(xp);
            bf16x4 yo;
#pragma unroll
            for (int i = 0; i < 4; ++i) yo[i] = (bf16)(rsc * (tt ? Y1[4 * q + i] : Y0[4 * q + i]) + d4[i] * (float)xv[i]);
            *reinterpret_cast<bf16x4*>(xp) = yo;
          } else {
            const f32x4 xv = *reinterpret_cast<const f32x4*>(xp);
            f32x4 yo;
#pragma unroll
            for (int i = 0; i < 4; ++i) yo[i] = rsc * (tt ? Y1[4 * q + i] : Y0[4 * q + i]) + d4[i] * xv[i];
            *reinterpret_cast<f32x4*>(xp) = yo;
          }
        }
      }
    };
    readout<TM, N>(H, sg.fr.ct, ll, Y0, Y1);
    float rs0, rs1;
    if (fact) {
      Y0 = mma(xa[0], sg.fr.cb[0][0][ll], Y0);
      Y0 = mma(xa[1], sg.fr.cb[0][1][ll], Y0);
      Y1 = mma(xa[0], sg.fr.cb[1][0][ll], Y1);
      Y1 = mma(xa[1], sg.fr.cb[1][1][ll], Y1);
      Y1 = mma(xa[2], sg.fr.cb[2][0][ll], Y1);
      Y1 = mma(xa[3], sg.fr.cb[2][1][ll], Y1);
      rs0 = __expf(kappa + cs0);
      rs1 = __expf(kappa + cs1);
      kappa += cse;
    } else {
      // exact path (kappa = 0 here): xa_s = dt_s x_s, each masked C B^T entry decayed by e^{cs_t - cs_s}
      // (s <= t), the state term weighted by e^{cs_t};  H <- e^{cse} H + B^T (e^{cse - cs} xa)
      Y0 *= __expf(cs0);
      Y1 *= __expf(cs1);
#pragma unroll
      for (int ti = 0; ti < 3; ++ti) {
        const int st = (ti == 2) ? 1 : 0;
        const float cst = (ti == 0) ? cs0 : cs1;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float css[8];
          kset_vals(sm.cs[w] + 32 * st, c, halfq, css);
          const Frag<TM> cb = sg.fr.cb[ti][c][ll];
          Frag<TM> md;
#pragma unroll
          for (int e = 0; e < 8; ++e) md.set(e, cb.get(e) * __expf(fminf(cst - css[e], 0.f)));
          if (ti == 0) Y0 = mma(xa[2 * st + c], md, Y0);
          else Y1 = mma(xa[2 * st + c], md, Y1);
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        float f[8];
        kset_vals(sm.cs[w], c, halfq, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) xa[c].set(e, xa[c].get(e) * __expf(cse - f[e]));
      }
      const float e = __expf(cse);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) H[nt] *= e;
      rs0 = rs1 = 1.f;
    }
    // state update (MFMA) and output epilogue (VALU, LDS) are independent: one block, interleaved
    state_update<TM, N>(H, sg.fr.bt, xa, ll);
    epilogue(rs0, rs1);
  }
  // y of the last segment
  {
    const int si = nseg - 1;
    const int cur = (NBUF == 2) ? (si & 1) : 0;
    const int pos = c0 + si * SEG;
    if (zg && !ZPRE) load_zhalf<T>(zg + (int64_t)pos * p.z_sl, p.z_sl, c1 - 1 - pos, l, zv);
    store_yhalf<T>(yg + (int64_t)pos * p.y_sl, p.y_sl, sm.st[cur].X[w], c1 - pos, l, zg != nullptr, zv);
  }
}

// ------------------------------------------------------------------ launch

size_t ssd_frag_bytes(int dtype, int dstate) {
  return dtype == DT_BF16 ? (dstate == 128 ? sizeof(SegFrags<bf16, 128>) : sizeof(SegFrags<bf16, 64>))
                          : (dstate == 128 ? sizeof(SegFrags<float, 128>) : sizeof(SegFrags<float, 64>));
}

// Workspace parts, each 256-byte aligned: chunk-local states (bf16 for bf16 I/O, fp32 otherwise), chunk
// log-decays, per-segment shared fragments, bf16 entering states (bf16 I/O only).
// The two-pass bf16 path (ssd_lookback.hip) needs no segment fragments, and bf16 entering states only when the
// scan does not sum them itself (more than LB_MAX chunks).
struct SsdWorkspace {
  size_t states, decay, frags, entering;
  size_t total() const { return align256(states) + align256(decay) + align256(frags) + align256(entering); }
};
static SsdWorkspace ssd_workspace(int batch, int seqlen, int nchunks, int nheads, int headdim, int dstate,
                                  int ngroups, int dtype) {
  const size_t nstate = (size_t)batch * nchunks * nheads * headdim * dstate;
  const size_t nseg = (size_t)(seqlen + SEG - 1) / SEG;
  const bool lb = ssd_lb_supported(dtype, dstate);
  SsdWorkspace w;
  w.states = nstate * (dtype == DT_BF16 ? sizeof(bf16) : sizeof(float));
  w.decay = (size_t)batch * nheads * nchunks * sizeof(float);
  w.frags = lb ? 0 : (size_t)batch * ngroups * nseg * ssd_frag_bytes(dtype, dstate);
  w.entering = (dtype == DT_BF16 && (!lb || nchunks > LB_MAX)) ? nstate * sizeof(bf16) : 0;
  return w;
}

size_t ssd_workspace_bytes(int batch, int seqlen, int nchunks, int nheads, int headdim, int dstate, int ngroups,
                           int dtype) {
  return ssd_workspace(batch, seqlen, nchunks, nheads, headdim, dstate, ngroups, dtype).total();
}

void ssd_workspace_layout(SsdParams& p, void* workspace) {
  const SsdWorkspace w = ssd_workspace(p.batch, p.seqlen, p.nchunks, p.nheads, p.headdim, p.dstate, p.ngroups,
                                       p.dtype);
  char* c = reinterpret_cast<char*>(workspace);
  p.chunk_states = reinterpret_cast<float*>(c);
  c += align256(w.states);
  p.chunk_decay = reinterpret_cast<float*>(c);
  c += align256(w.decay);
  p.seg_frags = w.frags ? c : nullptr;
  c += align256(w.frags);
  p.entering = w.entering ? c : nullptr;
}

template <typename T, typename TM, int N, int HG>
static hipError_t launch_ssd_t(const SsdParams& p, hipStream_t st) {
  hipLaunchKernelGGL((ssd_seg_frags_kernel<T, TM, N>), dim3((unsigned)p.nseg, (unsigned)p.ngroups, (unsigned)p.batch),
                     dim3(512), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 grid((unsigned)p.nchunks, (unsigned)(p.nheads / HG), (unsigned)p.batch);
  hipLaunchKernelGGL((ssd_chunk_state_kernel<T, TM, N, HG>), grid, dim3(128 * HG), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int per8 = HD * N / 8;
  dim3 g2((unsigned)((per8 + 255) / 256), (unsigned)(p.batch * p.nheads));
  hipLaunchKernelGGL((ssd_state_pass_kernel<T>), g2, dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_chunk_scan_kernel<T, TM, N, HG>), grid, dim3(128 * HG), 0, st, p);
  return hipGetLastError();
}

template <typename T, typename TM, int N, int HG>
constexpr bool ssd_fits = !(sizeof(T) == 4 && N == 128 && HG > 1) &&   // fp32 N=128 runs one head per workgroup
                          sizeof(ScanSmem<T, TM, N, HG, 1>) <= LDS_BYTES && sizeof(StateSmem<T, TM, N, HG, 1>) <= LDS_BYTES &&
                          bt_blocks<TM, N> % (2 * HG) == 0 && Tile<T, N>::NBLK % (2 * HG) == 0;

template <typename T, typename TM, int N>
static hipError_t launch_ssd_n(const SsdParams& p, hipStream_t st) {
  switch (p.heads_per_wg) {
    case 4:
      if constexpr (ssd_fits<T, TM, N, 4>) return launch_ssd_t<T, TM, N, 4>(p, st);
      return hipErrorInvalidValue;
    case 2:
      if constexpr (ssd_fits<T, TM, N, 2>) return launch_ssd_t<T, TM, N, 2>(p, st);
      return hipErrorInvalidValue;
    case 1:
      if constexpr (ssd_fits<T, TM, N, 1>) return launch_ssd_t<T, TM, N, 1>(p, st);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

// Empty sequence: the final state is the initial state (or zero) -- a plain kernel rather than a memset or
// copy node, so the launch behaves the same inside a captured graph.
__global__ __launch_bounds__(256) void ssd_empty_kernel(const float* __restrict__ h0, float* __restrict__ fin, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) fin[i] = h0 ? h0[i] : 0.f;
}

hipError_t launch_ssd_state_pass(const SsdParams& p, hipStream_t st) {
  const int per8 = HD * p.dstate / 8;
  dim3 g2((unsigned)((per8 + 255) / 256), (unsigned)(p.batch * p.nheads));
  if (p.dtype == DT_BF16) hipLaunchKernelGGL((ssd_state_pass_kernel<bf16>), g2, dim3(256), 0, st, p);
  else hipLaunchKernelGGL((ssd_state_pass_kernel<float>), g2, dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_ssd(const SsdParams& p, hipStream_t st) {
  if (p.nchunks == 0) {
    if (!p.final_state) return hipSuccess;
    const size_t n = (size_t)p.batch * p.nheads * HD * p.dstate;
    hipLaunchKernelGGL(ssd_empty_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.init_state,
                       p.final_state, n);
    return hipGetLastError();
  }
  if (ssd_lb_supported(p.dtype, p.dstate)) return launch_ssd_lb(p, st);    // its scan writes xsum itself
  hipError_t e = hipErrorInvalidValue;
  if (p.dtype == DT_BF16) {
    if (p.dstate == 128) e = launch_ssd_n<bf16, bf16, 128>(p, st);
    if (p.dstate == 64) e = launch_ssd_n<bf16, bf16, 64>(p, st);
  } else {
    if (p.dstate == 128) e = launch_ssd_n<float, float, 128>(p, st);
    if (p.dstate == 64) e = launch_ssd_n<float, float, 64>(p, st);
  }
  if (e == hipSuccess && p.xsum) e = launch_ssd_xsum(p, st);
  return e;
}

// xsum[b][t][h][half] = sum of x[b][t][h][32 half .. 32 half + 31]: one (token, head, half) per thread.
template <typename T>
__global__ __launch_bounds__(256) void ssd_xsum_kernel(SsdParams p) {
  const int64_t n = (int64_t)p.batch * p.seqlen * p.nheads * 2;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int half = (int)(i & 1), h = (int)((i >> 1) % p.nheads);
  const int64_t bt = (i >> 1) / p.nheads, t = bt % p.seqlen, b = bt / p.seqlen;
  const T* row = reinterpret_cast<const T*>(p.x) + b * p.x_sb + t * p.x_sl + (int64_t)h * p.x_sh + 32 * half;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 32; ++k) s += to_f32(row[k]);
  p.xsum[i] = s;
}

hipError_t launch_ssd_xsum(const SsdParams& p, hipStream_t st) {
  const int64_t n = (int64_t)p.batch * p.seqlen * p.nheads * 2;
  if (n == 0) return hipSuccess;
  const unsigned nb = (unsigned)((n + 255) / 256);
  if (p.dtype == DT_BF16) hipLaunchKernelGGL(ssd_xsum_kernel<bf16>, dim3(nb), dim3(256), 0, st, p);
  else hipLaunchKernelGGL(ssd_xsum_kernel<float>, dim3(nb), dim3(256), 0, st, p);
  return hipGetLastError();
}

}  // namespace mh
