// Mamba-2 SSD chunked-scan prefill for gfx950.
//
// Recurrence (per batch b, head h with group g = h / (H/G), channel p, state n):
//     h_t = exp(A_h dt_t) h_{t-1} + dt_t x_t[p] B_t[g, n]
//     y_t[p] = sum_n C_t[g, n] h_t[p, n] + D x_t[p]
// i.e. the reference's selective_scan (mamformer/layers/mamba2.py:84-126) in the
// per-head SSD parameterisation, with an optional initial state (prefill of a
// cached sequence) and the final state returned for the decode cache.
//
// Decomposition (three launches on the caller's stream):
//   1. ssd_chunk_state  grid (nchunks, H/HG, b): for each state chunk of
//      `chunk_len` tokens the chunk-local final state
//          S_k[p, n] = sum_{s in k} exp(sum_{s<tau in k} A dt_tau) dt_s x_s[p] B_s[n]
//      as an MFMA reduction over tokens, plus the chunk's total log-decay.
//   2. ssd_state_pass   elementwise over (b, h, P*N): H_0 = h0, H_{k+1} = e^{T_k} H_k + S_k.
//      Writes the *entering* state H_k over S_k and the final state.
//   3. ssd_chunk_scan   grid (nchunks, H/HG, b): each head's state chunk is
//      walked in segments of <= 64 tokens with the running state in MFMA
//      accumulator registers, kept as H = e^kappa * Hs (Hs fp32, kappa a scalar).
//      With cs the in-segment cumulative log-decay counted from just after the
//      segment's first token (cs_0 = 0, first-token decay folded into kappa):
//          xs_s = e^{-kappa - cs_s} dt_s x_s                      (one bf16 operand per token)
//          Y    = [C B^T o causal mask] xs + C Hs^T                (MFMA; no per-segment state rescale)
//          y_t  = e^{cs_t + kappa} Y_t + D x_t
//          Hs  += B^T xs ;  kappa += cs_end
//      exp(cs_t - cs_s) = e^{cs_t + kappa} e^{-kappa - cs_s} is exact; segments
//      are cut so the spread of cs stays <= RANGE, and Hs is renormalised
//      (Hs *= e^kappa, kappa = 0) whenever a factor would leave e^{+-RANGE}, so
//      every intermediate stays finite for any decay.
// Work split: a workgroup owns HG heads of one group with two waves per head;
// wave w handles head w / 2 and the 32 state columns p of half w % 2, so each
// wave's state is N/32 accumulator tiles.  C B^T (three 32x32 tiles) and the
// B^T fragments are computed once per segment and shared by all waves.
// Transposes needed by the token-contracted MFMAs (B^T, x^T) are done on the
// MFMA unit itself: a row-loaded tile times an identity fragment lands in the
// accumulator layout that the next MFMA consumes.
// Memory: tiles of the next segment are fetched straight into a second LDS
// buffer (global_load_lds_dwordx4, no register staging) while the current one
// is computed; LDS tiles are XOR-swizzled per row for conflict-free fragment
// reads; y is staged in LDS and written with 16-byte stores; the chunk-state
// workspace is kept in MFMA fragment order (64 contiguous bytes per lane).
// bf16 I/O uses 32x32x16 bf16 MFMAs, fp32 I/O 32x32x2 fp32 MFMAs; accumulation is fp32.
#include "common.h"
#include "launch.h"

namespace mh {

constexpr int SEG = 64;          // tokens per segment (max)
constexpr int HD = 64;           // headdim handled by these kernels
constexpr float RANGE = 40.f;    // max spread of in-segment cumulative log-decay; renormalisation threshold

// ------------------------------------------------------------------ wave helpers

// Reverse inclusive prefix sum over the 64 lanes: r_l = sum_{i >= l} v_i.
__device__ __forceinline__ float wave_incl_rscan(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_down(v, off, 64);
    if (l + off < 64) v += o;
  }
  return v;
}
__device__ __forceinline__ float wave_prefix_max(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (l >= off) v = fmaxf(v, o);
  }
  return v;
}
__device__ __forceinline__ float wave_prefix_min(float v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    float o = __shfl_up(v, off, 64);
    if (l >= off) v = fminf(v, o);
  }
  return v;
}

__device__ __forceinline__ float process_dt(const SsdParams& p, float dt, int h) {
  if (p.dt_bias) dt += p.dt_bias[h];
  if (p.dt_softplus) dt = softplus_f(dt);
  if (p.has_dt_limit) dt = fminf(fmaxf(dt, p.dt_min), p.dt_max);
  return dt;
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------------ LDS tiles

// Rows of W elements, unpadded, 16-byte chunks XOR-swizzled by row (chunk c of
// row r lives at chunk c ^ (r & MASK)) so the lanes of one LDS access phase,
// reading the same column of consecutive rows, hit distinct banks.
template <typename T, int W>
struct Tile {
  static constexpr int EPC = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  static constexpr int CPR = W / EPC;               // chunks per row (power of two)
  static constexpr int MASK = (CPR < 16 ? CPR : 16) - 1;
  static constexpr int RPB = 64 / CPR;              // rows per 1 KB block (one wave-wide direct load)
  static constexpr int NBLK = SEG / RPB;            // 1 KB blocks per tile
  __device__ static __forceinline__ int chunk(int r, int c) { return r * W + (c ^ (r & MASK)) * EPC; }
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// Direct global -> LDS fetch of 1 KB blocks [blk0, blk0 + nblk) of a swizzled
// tile: lane i of the wave writes LDS bytes [16 i, 16 i + 16) of the block, so
// it fetches the logical chunk that the swizzle places there.  Rows past
// `last_tok` (end of the sequence) re-read the last valid row; their values
// are finite and every consumer masks them.
template <typename T, int W>
__device__ __forceinline__ void fetch_tile(T* dst, const T* src, int64_t row_stride, int tok0, int last_tok,
                                           int blk0, int nblk, int lane) {
  using TL = Tile<T, W>;
  const int rr = lane / TL::CPR, phys = lane % TL::CPR;
  for (int q = 0; q < nblk; ++q) {
    const int blk = blk0 + q;
    const int r = blk * TL::RPB + rr;
    const int c = phys ^ (r & TL::MASK);
    const int tok = min(tok0 + r, last_tok);
    const T* g = src + (int64_t)tok * row_stride + c * TL::EPC;
    T* d = dst + blk * (1024 / (int)sizeof(T));
    __builtin_amdgcn_global_load_lds((glb_void_t*)g, (lds_void_t*)d, 16, 0, 0);
  }
}

// 8 consecutive elements of row r starting at column e0 (e0 % 8 == 0) as an MFMA fragment.
template <typename TM, typename T, int W>
__device__ __forceinline__ Frag<TM> row_frag(const T* tile, int r, int e0) {
  Frag<TM> f;
  if constexpr (sizeof(T) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(tile + Tile<T, W>::chunk(r, e0 / 8));
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + Tile<T, W>::chunk(r, e0 / 4));
    const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + Tile<T, W>::chunk(r, e0 / 4 + 1));
#pragma unroll
    for (int j = 0; j < 4; ++j) { f.v[j] = lo[j]; f.v[4 + j] = hi[j]; }
  }
  return f;
}
// KSET fragment of row r (base % 16 == 0): columns base+4*half+{0..3} and base+8+4*half+{0..3}.
template <typename TM, typename T, int W>
__device__ __forceinline__ Frag<TM> kset_frag(const T* tile, int r, int base, int half) {
  Frag<TM> f;
  if constexpr (sizeof(T) == 2) {
    const bf16x4 lo = *reinterpret_cast<const bf16x4*>(tile + Tile<T, W>::chunk(r, base / 8) + 4 * half);
    const bf16x4 hi = *reinterpret_cast<const bf16x4*>(tile + Tile<T, W>::chunk(r, base / 8 + 1) + 4 * half);
#pragma unroll
    for (int j = 0; j < 4; ++j) { f.v[j] = lo[j]; f.v[4 + j] = hi[j]; }
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + Tile<T, W>::chunk(r, base / 4 + half));
    const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + Tile<T, W>::chunk(r, base / 4 + 2 + half));
#pragma unroll
    for (int j = 0; j < 4; ++j) { f.v[j] = lo[j]; f.v[4 + j] = hi[j]; }
  }
  return f;
}

// Per-token scale factors of the 8 tokens a KSET fragment covers (k-step c):
// tokens 16c+4*half+{0..3} and 16c+8+4*half+{0..3}, read as two float4.
__device__ __forceinline__ void kset_scales(const float* v, int c, int half, float (&s)[8]) {
  const f32x4 lo = *reinterpret_cast<const f32x4*>(v + 16 * c + 4 * half);
  const f32x4 hi = *reinterpret_cast<const f32x4*>(v + 16 * c + 8 + 4 * half);
#pragma unroll
  for (int j = 0; j < 4; ++j) { s[j] = lo[j]; s[4 + j] = hi[j]; }
}

// Identity B-operand fragment for k-step c of a 32-wide block: element j has
// k = 16c + 8*half + j, the lane's column is l32.
template <typename TM>
__device__ __forceinline__ Frag<TM> ident_frag(int c, int half, int l32) {
  Frag<TM> f;
#pragma unroll
  for (int j = 0; j < 8; ++j) f.set(j, (16 * c + 8 * half + j == l32) ? 1.f : 0.f);
  return f;
}

// Transpose a 32x32 block of a row-major LDS tile through the MFMA unit:
// returns the accumulator tile D[r][q] = tile[r0 + r][q0 + q] (r, q < 32), whose
// lane l holds column q0 + (l % 32) and rows r0 + acc_row(half, i).
template <typename TM, typename T, int W>
__device__ __forceinline__ f32x16 mfma_transpose(const T* tile, int r0, int q0, const Frag<TM> (&id)[2], int half,
                                                 int l32) {
  f32x16 acc = zero16();
#pragma unroll
  for (int c = 0; c < 2; ++c) acc = mma(row_frag<TM, T, W>(tile, r0 + l32, q0 + 16 * c + 8 * half), id[c], acc);
  return acc;
}

// x~^T fragments of one 32-column p-tile: lane = p, elements = tokens (KSET), each token scaled.
template <typename TM, typename T>
__device__ __forceinline__ void scaled_xt_frags(const T* xtile, int pt, const float* scale, const Frag<TM> (&id)[2],
                                                int half, int l32, Frag<TM> (&xf)[4]) {
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const f32x16 xt = mfma_transpose<TM, T, HD>(xtile, 32 * st, 32 * pt, id, half, l32);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float sc[8];
      kset_scales(scale, 2 * st + c, half, sc);
#pragma unroll
      for (int j = 0; j < 8; ++j) xf[2 * st + c].set(j, xt[8 * c + j] * sc[j]);
    }
  }
}

// Shared per-segment MFMA work of a workgroup of NW waves: the three C B^T
// tiles (N/16 MFMAs each, k-reductions, one wave each) and the 2 * N/32 B^T
// blocks (2 MFMAs each), spread so the busiest wave does one C B^T tile.
template <int NW, int N>
struct SharedWork {
  static constexpr int NBLK = 2 * (N / 32);
  static constexpr int CBW = NW < 3 ? NW : 3;                   // waves that own C B^T tiles
  static constexpr int BTW = NW > 3 ? NW - 3 : NW;              // waves that own B^T blocks
  static constexpr int BTPER = (NBLK + BTW - 1) / BTW;
  static constexpr int CBPER = (3 + CBW - 1) / CBW;
  __device__ static __forceinline__ int cb_tile(int w, int i) { return (w < CBW) ? w + i * CBW : 99; }
  __device__ static __forceinline__ int bt_block(int w, int i) {
    if (NW > 3) return (w >= 3) ? (w - 3) + i * BTW : 99;
    return w + i * NW;
  }
};

// B^T A-operand fragments (row n, k = token via KSET) of the B tile, computed
// by the waves SharedWork assigns, in registers until the caller's barrier.
template <typename T, typename TM, int N, int NW>
struct BtWork {
  using SW = SharedWork<NW, N>;
  f32x16 acc[SW::BTPER];
  __device__ __forceinline__ void compute(const T* Bs, int w, const Frag<TM> (&id)[2], int half, int l32) {
#pragma unroll
    for (int i = 0; i < SW::BTPER; ++i) {
      const int blk = SW::bt_block(w, i);
      if (blk < SW::NBLK) acc[i] = mfma_transpose<TM, T, N>(Bs, 32 * (blk & 1), 32 * (blk >> 1), id, half, l32);
    }
  }
  __device__ __forceinline__ void store(Frag<TM> (*Bt)[4][64], int w, int l) const {
#pragma unroll
    for (int i = 0; i < SW::BTPER; ++i) {
      const int blk = SW::bt_block(w, i);
      if (blk < SW::NBLK) {
        Bt[blk >> 1][2 * (blk & 1)][l] = acc_to_frag<TM>(acc[i], 0);
        Bt[blk >> 1][2 * (blk & 1) + 1][l] = acc_to_frag<TM>(acc[i], 1);
      }
    }
  }
};

// One buffer of segment tiles.  The B tile is overwritten by its B^T fragments
// once both have been read (same size: 64 x N elements).
template <typename T, typename TM, int N, int HG>
struct SegTiles {
  union {
    T B[SEG * N];
    Frag<TM> Bt[N / 32][4][64];
  };
  T C[SEG * N];
  T X[HG][SEG * HD];
};
template <typename T, typename TM, int N, int HG>
struct StateTiles {
  union {
    T B[SEG * N];
    Frag<TM> Bt[N / 32][4][64];
  };
  T X[HG][SEG * HD];
};
static_assert(sizeof(Frag<bf16>) * (128 / 32) * 4 * 64 == sizeof(bf16) * SEG * 128, "Bt must alias B exactly");
static_assert(sizeof(Frag<float>) * (128 / 32) * 4 * 64 == sizeof(float) * SEG * 128, "Bt must alias B exactly");

template <typename T, typename TM, int N, int HG, int NBUF>
struct ScanSmem {
  SegTiles<T, TM, N, HG> buf[NBUF];
  Frag<TM> CB[3][2][64];          // masked (C B^T)^T tiles as B-operand fragments: tile, k-step, lane
  float cs[HG][SEG];              // log of the output row scale
  float sa[HG][SEG];              // per-token operand scale
  float dcol[HG][HD];             // D per column of each head (per-head D broadcast)
  int len[HG];
};
template <typename T, typename TM, int N, int HG, int NBUF>
struct StateSmem {
  StateTiles<T, TM, N, HG> buf[NBUF];
  float w[HG][SEG];
};

// Tiles are double-buffered (the next segment fetched during this one's
// compute) where two buffers fit in the 160 KB of LDS, else single-buffered
// (fetched between segments).
constexpr size_t LDS_BYTES = 160 * 1024;
template <typename T, typename TM, int N, int HG>
constexpr int scan_nbuf = sizeof(ScanSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1;
template <typename T, typename TM, int N, int HG>
constexpr int state_nbuf = sizeof(StateSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1;

// Offset (floats) of state tile (nt, pt) element block of lane l in the fragment-native workspace order.
__device__ __forceinline__ int frag_off(int nt, int pt, int l) { return ((nt * 2 + pt) * 64 + l) * 16; }

// Fetch the B (and optionally C) tiles shared by the workgroup and the x tile
// of each head (by that head's two waves) for the segment starting at tok0.
template <typename T, int N, int NW>
__device__ __forceinline__ void fetch_segment(T* Bs, T* Cs, T* Xs, const T* Bg, int64_t B_sl, const T* Cg,
                                              int64_t C_sl, const T* xg, int64_t x_sl, int tok0, int last_tok,
                                              int w, int ph, int l) {
  using TB = Tile<T, N>;
  using TX = Tile<T, HD>;
  constexpr int BPW = (TB::NBLK + NW - 1) / NW;             // B/C blocks per wave
  const int b0 = w * BPW, nb = max(0, min(BPW, TB::NBLK - b0));
  fetch_tile<T, N>(Bs, Bg, B_sl, tok0, last_tok, b0, nb, l);
  if (Cs) fetch_tile<T, N>(Cs, Cg, C_sl, tok0, last_tok, b0, nb, l);
  constexpr int XPW = TX::NBLK / 2;                         // x blocks per wave (two waves per head)
  fetch_tile<T, HD>(Xs, xg, x_sl, tok0, last_tok, ph * XPW, XPW, l);
}

// ------------------------------------------------------------------ kernel 1

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(128 * HG) void ssd_chunk_state_kernel(SsdParams p) {
  constexpr int NBUF = state_nbuf<T, TM, N, HG>;
  using SM = StateSmem<T, TM, N, HG, NBUF>;
  __shared__ SM sm;
  constexpr int NT = N / 32, NW = 2 * HG;
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int j = w >> 1, ph = w & 1;
  const int h = blockIdx.y * HG + j;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const float Ah = p.A[h];
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);

  f32x16 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = zero16();

  // Walk the chunk backwards so the decay to the chunk end is a running suffix
  // sum; the previous segment's tiles are fetched while this one is reduced.
  float suffix = 0.f;
  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  int cur = 0;
  float dtraw = 0.f;
  {
    const int pos = c0 + (nseg - 1) * SEG;
    fetch_segment<T, N, NW>(sm.buf[0].B, nullptr, sm.buf[0].X[j], Bg, p.B_sl, nullptr, 0, xg, p.x_sl, pos, c1 - 1,
                            w, ph, l);
    if (pos + l < c1) dtraw = dtg[(int64_t)(pos + l) * p.dt_sl];
    wait_vmem();
    __syncthreads();
  }
  for (int si = nseg - 1; si >= 0; --si) {
    auto& bf = sm.buf[cur];
    const int pos = c0 + si * SEG;
    const int t = pos + l;
    const float dtv = (t < c1) ? process_dt(p, dtraw, h) : 0.f;
    const float a = Ah * dtv;
    const float rs = wave_incl_rscan(a);                 // sum_{i >= l} a_i within segment
    float ex = __shfl_down(rs, 1, 64);                    // sum_{i > l}
    if (l == 63) ex = 0.f;
    if (ph == 0) sm.w[j][l] = __expf(ex + suffix) * dtv;
    suffix += __shfl(rs, 0, 64);
    if (si > 0) {                                          // fetch the previous segment
      const int pp = pos - SEG;
      if constexpr (NBUF == 2)
        fetch_segment<T, N, NW>(sm.buf[cur ^ 1].B, nullptr, sm.buf[cur ^ 1].X[j], Bg, p.B_sl, nullptr, 0, xg,
                                p.x_sl, pp, c1 - 1, w, ph, l);
      dtraw = dtg[(int64_t)(pp + l) * p.dt_sl];
    }
    BtWork<T, TM, N, NW> bt;
    bt.compute(bf.B, w, id, half, l32);
    __syncthreads();
    bt.store(bf.Bt, w, l);
    __syncthreads();
    Frag<TM> xf[4];
    scaled_xt_frags<TM, T>(bf.X[j], ph, sm.w[j], id, half, l32, xf);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      Frag<TM> btf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) btf[c] = bf.Bt[nt][c][l];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[nt] = mma(btf[c], xf[c], acc[nt]);
    }
    if constexpr (NBUF == 1) {
      __syncthreads();
      if (si > 0)
        fetch_segment<T, N, NW>(sm.buf[0].B, nullptr, sm.buf[0].X[j], Bg, p.B_sl, nullptr, 0, xg, p.x_sl, pos - SEG,
                                c1 - 1, w, ph, l);
    }
    wait_vmem();
    __syncthreads();
    cur ^= NBUF - 1;
  }

  float* out = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    f32x4* o4 = reinterpret_cast<f32x4*>(out + frag_off(nt, ph, l));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 v;
      v[0] = acc[nt][4 * q]; v[1] = acc[nt][4 * q + 1]; v[2] = acc[nt][4 * q + 2]; v[3] = acc[nt][4 * q + 3];
      o4[q] = v;
    }
  }
  if (l == 0 && ph == 0) p.chunk_decay[((int64_t)b * p.nheads + h) * p.nchunks + k] = suffix;
}

// ------------------------------------------------------------------ kernel 2

// Workspace element e (fragment-native order) <-> canonical state index p * N + n.
__device__ __forceinline__ int canon_index(int e, int N) {
  const int r = e & 15, lane = (e >> 4) & 63, tile = e >> 10;
  const int pt = tile & 1, nt = tile >> 1;
  return (32 * pt + (lane & 31)) * N + 32 * nt + acc_row(lane >> 5, r);
}

__global__ __launch_bounds__(256) void ssd_state_pass_kernel(SsdParams p) {
  const int bh = blockIdx.y;
  const int b = bh / p.nheads, h = bh - b * p.nheads;
  const int per = HD * p.dstate;                  // state elements per (b, h)
  const int e4 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (e4 >= per) return;
  const int ci = canon_index(e4, p.dstate);       // 4 consecutive e map to 4 consecutive canonical n
  f32x4 H;
  H[0] = H[1] = H[2] = H[3] = 0.f;
  if (p.init_state) H = *reinterpret_cast<const f32x4*>(p.init_state + (int64_t)bh * per + ci);
  const float* dec = p.chunk_decay + (int64_t)bh * p.nchunks;
  for (int k = 0; k < p.nchunks; ++k) {
    float* sp = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * per + e4;
    const f32x4 S = *reinterpret_cast<const f32x4*>(sp);
    *reinterpret_cast<f32x4*>(sp) = H;
    const float a = __expf(dec[k]);
#pragma unroll
    for (int i = 0; i < 4; ++i) H[i] = a * H[i] + S[i];
  }
  if (p.final_state) *reinterpret_cast<f32x4*>(p.final_state + (int64_t)bh * per + ci) = H;
}

// ------------------------------------------------------------------ kernel 3

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(128 * HG) void ssd_chunk_scan_kernel(SsdParams p) {
  constexpr int NBUF = scan_nbuf<T, TM, N, HG>;
  using SM = ScanSmem<T, TM, N, HG, NBUF>;
  using SW = SharedWork<2 * HG, N>;
  using TX = Tile<T, HD>;
  __shared__ SM sm;
  constexpr int NT = N / 32, NW = 2 * HG;
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int j = w >> 1, ph = w & 1;                       // head of the workgroup, 32-column half of P
  const int h = blockIdx.y * HG + j;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const int last = p.seqlen - 1;
  const float Ah = p.A[h];
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const T* Cg = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  T* yg = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh;
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);
  if (ph == 0) sm.dcol[j][l] = p.D ? (p.D_per_channel ? p.D[h * HD + l] : p.D[h]) : 0.f;

  // Entering state H_k (fragment-native workspace order), columns of this wave's P-half;
  // H = e^kappa * Hs with kappa = 0.
  f32x16 Hs[NT];
  {
    const float* hk = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const f32x4* h4 = reinterpret_cast<const f32x4*>(hk + frag_off(nt, ph, l));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = h4[q];
        Hs[nt][4 * q] = v[0]; Hs[nt][4 * q + 1] = v[1]; Hs[nt][4 * q + 2] = v[2]; Hs[nt][4 * q + 3] = v[3];
      }
    }
  }
  float kappa = 0.f;

  int cur = 0;
  float dtraw = (c0 + l < c1) ? dtg[(int64_t)(c0 + l) * p.dt_sl] : 0.f;
  fetch_segment<T, N, NW>(sm.buf[0].B, sm.buf[0].C, sm.buf[0].X[j], Bg, p.B_sl, Cg, p.C_sl, xg, p.x_sl, c0, last,
                          w, ph, l);
  wait_vmem();
  __syncthreads();

  for (int pos = c0; pos < c1;) {
    auto& bf = sm.buf[cur];
    // ---- dt, in-segment cumulative log-decay, longest admissible prefix (both waves of a head agree)
    const int t = pos + l;
    const float dtv = (t < c1) ? process_dt(p, dtraw, h) : 0.f;
    const float csa = wave_incl_scan(Ah * dtv);            // includes token 0's own decay
    const float pmax = wave_prefix_max(csa), pmin = wave_prefix_min(csa);
    const bool ok = (pmax - pmin <= RANGE) && (t < c1);
    const uint64_t bal = __ballot(ok);
    const int len_w = (~bal == 0ull) ? 64 : __builtin_ctzll(~bal);
    if (l == 0 && ph == 0) sm.len[j] = len_w;
    __syncthreads();

    int len = sm.len[0];
#pragma unroll
    for (int i = 1; i < HG; ++i) len = min(len, sm.len[i]);
    const int next = pos + len;
    if (next < c1) {                                       // fetch the next segment into the other buffer
      if constexpr (NBUF == 2) {
        auto& nb = sm.buf[cur ^ 1];
        fetch_segment<T, N, NW>(nb.B, nb.C, nb.X[j], Bg, p.B_sl, Cg, p.C_sl, xg, p.x_sl, next, last, w, ph, l);
      }
      dtraw = (next + l < c1) ? dtg[(int64_t)(next + l) * p.dt_sl] : 0.f;
    }
    const float a0 = __shfl(csa, 0, 64);
    const float cs = csa - a0;                             // cs_0 = 0
    const float csmax = __shfl(pmax, len - 1, 64) - a0, csmin = __shfl(pmin, len - 1, 64) - a0;
    float ke = kappa + a0;                                 // kappa with token 0's decay applied
    if (ke + csmin < -RANGE || ke + csmax > RANGE) {       // renormalise Hs (wave-uniform)
      const float s = __expf(ke);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) Hs[nt] *= s;
      ke = 0.f;
    }
    if (ph == 0) {
      sm.cs[j][l] = cs + ke;
      sm.sa[j][l] = (l < len) ? __expf(-ke - cs) * dtv : 0.f;
    }

    // ---- shared: C B^T tiles (s-tile, t-tile) in {(0,0), (0,1), (1,1)} and B^T fragments;
    //      both read the B tile, which the B^T fragments overwrite after the barrier
    f32x16 cbacc[SW::CBPER];
#pragma unroll
    for (int i = 0; i < SW::CBPER; ++i) {
      const int ti = SW::cb_tile(w, i);
      cbacc[i] = zero16();
      if (ti < 3) {
        const int st = (ti == 2) ? 1 : 0, tt = (ti == 0) ? 0 : 1;
#pragma unroll
        for (int c = 0; c < N / 16; ++c)
          cbacc[i] = mma(row_frag<TM, T, N>(bf.B, 32 * st + l32, 16 * c + 8 * half),
                         row_frag<TM, T, N>(bf.C, 32 * tt + l32, 16 * c + 8 * half), cbacc[i]);
      }
    }
    BtWork<T, TM, N, NW> bt;
    bt.compute(bf.B, w, id, half, l32);
    __syncthreads();
    bt.store(bf.Bt, w, l);
#pragma unroll
    for (int i = 0; i < SW::CBPER; ++i) {
      const int ti = SW::cb_tile(w, i);
      if (ti < 3) {
        const int st = (ti == 2) ? 1 : 0, tt = (ti == 0) ? 0 : 1;
        const int tl = 32 * tt + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int s = 32 * st + acc_row(half, r);
          if (!(s <= tl && s < len)) cbacc[i][r] = 0.f;
        }
        sm.CB[ti][0][l] = acc_to_frag<TM>(cbacc[i], 0);
        sm.CB[ti][1][l] = acc_to_frag<TM>(cbacc[i], 1);
      }
    }
    __syncthreads();

    // ---- per wave: head j, p-tile ph
    Frag<TM> xf[4];
    scaled_xt_frags<TM, T>(bf.X[j], ph, sm.sa[j], id, half, l32, xf);
    // Y^T[p][t] = sum_s xs^T[p][s] M^T[s][t] + sum_n Hs[p][n] C^T[n][t]
    f32x16 Y0 = zero16(), Y1 = zero16();
    Y0 = mma(xf[0], sm.CB[0][0][l], Y0);
    Y0 = mma(xf[1], sm.CB[0][1][l], Y0);
    Y1 = mma(xf[0], sm.CB[1][0][l], Y1);
    Y1 = mma(xf[1], sm.CB[1][1][l], Y1);
    Y1 = mma(xf[2], sm.CB[2][0][l], Y1);
    Y1 = mma(xf[3], sm.CB[2][1][l], Y1);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const Frag<TM> hf = acc_to_frag<TM>(Hs[nt], c);
        Y0 = mma(hf, kset_frag<TM, T, N>(bf.C, l32, 32 * nt + 16 * c, half), Y0);
        Y1 = mma(hf, kset_frag<TM, T, N>(bf.C, 32 + l32, 32 * nt + 16 * c, half), Y1);
      }
    // y[t][p] = e^{cs_t + kappa} Y + D x, staged in place of x (this wave's 32 columns only)
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tl = 32 * tt + l32;
      const float rsc = __expf(sm.cs[j][tl]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p0 = 32 * ph + 8 * q + 4 * half;       // 4 consecutive columns, inside one 16-byte chunk
        T* xp = bf.X[j] + TX::chunk(tl, p0 / TX::EPC) + (p0 % TX::EPC);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.dcol[j][p0]);
        const float y0 = (tt ? Y1[4 * q] : Y0[4 * q]), y1 = (tt ? Y1[4 * q + 1] : Y0[4 * q + 1]);
        const float y2 = (tt ? Y1[4 * q + 2] : Y0[4 * q + 2]), y3 = (tt ? Y1[4 * q + 3] : Y0[4 * q + 3]);
        if constexpr (sizeof(T) == 2) {
          const bf16x4 xv = *reinterpret_cast<const bf16x4*>(xp);
          bf16x4 yv;
          yv[0] = (bf16)(rsc * y0 + d4[0] * (float)xv[0]);
          yv[1] = (bf16)(rsc * y1 + d4[1] * (float)xv[1]);
          yv[2] = (bf16)(rsc * y2 + d4[2] * (float)xv[2]);
          yv[3] = (bf16)(rsc * y3 + d4[3] * (float)xv[3]);
          *reinterpret_cast<bf16x4*>(xp) = yv;
        } else {
          const f32x4 xv = *reinterpret_cast<const f32x4*>(xp);
          f32x4 yv;
          yv[0] = rsc * y0 + d4[0] * xv[0];
          yv[1] = rsc * y1 + d4[1] * xv[1];
          yv[2] = rsc * y2 + d4[2] * xv[2];
          yv[3] = rsc * y3 + d4[3] * xv[3];
          *reinterpret_cast<f32x4*>(xp) = yv;
        }
      }
    }
    // ---- coalesced store of this wave's staged y columns for rows t < len
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int HCPR = TX::CPR / 2;                       // 16-byte chunks per row in a 32-column half
#pragma unroll
    for (int i = 0; i < SEG * HCPR / 64; ++i) {
      const int e = l + 64 * i;
      const int r = e / HCPR, c = ph * HCPR + (e - r * HCPR);
      if (r < len)
        *reinterpret_cast<uint4*>(yg + (int64_t)(pos + r) * p.y_sl + c * TX::EPC) =
            *reinterpret_cast<const uint4*>(bf.X[j] + TX::chunk(r, c));
    }
    __builtin_amdgcn_sched_barrier(0);
    // ---- state: Hs += B^T xs
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      Frag<TM> btf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) btf[c] = bf.Bt[nt][c][l];
#pragma unroll
      for (int c = 0; c < 4; ++c) Hs[nt] = mma(btf[c], xf[c], Hs[nt]);
    }
    kappa = ke + __shfl(cs, len - 1, 64);
    if constexpr (NBUF == 1) {
      __syncthreads();
      if (next < c1)
        fetch_segment<T, N, NW>(bf.B, bf.C, bf.X[j], Bg, p.B_sl, Cg, p.C_sl, xg, p.x_sl, next, last, w, ph, l);
    }
    wait_vmem();
    __syncthreads();
    cur ^= NBUF - 1;
    pos = next;
  }
}

// ------------------------------------------------------------------ launch

size_t ssd_workspace_bytes(int batch, int nchunks, int nheads, int headdim, int dstate) {
  const size_t states = (size_t)batch * nchunks * nheads * headdim * dstate * sizeof(float);
  const size_t decay = (size_t)batch * nheads * nchunks * sizeof(float);
  return ((states + 255) / 256) * 256 + ((decay + 255) / 256) * 256;
}

template <typename T, typename TM, int N, int HG>
static hipError_t launch_ssd_t(const SsdParams& p, hipStream_t st) {
  dim3 grid((unsigned)p.nchunks, (unsigned)(p.nheads / HG), (unsigned)p.batch);
  hipLaunchKernelGGL((ssd_chunk_state_kernel<T, TM, N, HG>), grid, dim3(128 * HG), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int per4 = HD * N / 4;
  dim3 g2((unsigned)((per4 + 255) / 256), (unsigned)(p.batch * p.nheads));
  hipLaunchKernelGGL(ssd_state_pass_kernel, g2, dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((ssd_chunk_scan_kernel<T, TM, N, HG>), grid, dim3(128 * HG), 0, st, p);
  return hipGetLastError();
}

template <typename T, typename TM, int N>
static hipError_t launch_ssd_n(const SsdParams& p, hipStream_t st) {
  switch (p.heads_per_wg) {
    case 4: return launch_ssd_t<T, TM, N, 4>(p, st);
    case 2: return launch_ssd_t<T, TM, N, 2>(p, st);
    case 1: return launch_ssd_t<T, TM, N, 1>(p, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_ssd(const SsdParams& p, hipStream_t st) {
  if (p.nchunks == 0) {
    // Empty sequence: the final state is the initial state.
    if (!p.final_state) return hipSuccess;
    const size_t bytes = (size_t)p.batch * p.nheads * HD * p.dstate * sizeof(float);
    if (p.init_state) return hipMemcpyAsync(p.final_state, p.init_state, bytes, hipMemcpyDeviceToDevice, st);
    return hipMemsetAsync(p.final_state, 0, bytes, st);
  }
  if (p.dtype == DT_BF16) {
    if (p.dstate == 128) return launch_ssd_n<bf16, bf16, 128>(p, st);
    if (p.dstate == 64) return launch_ssd_n<bf16, bf16, 64>(p, st);
  } else {
    if (p.dstate == 128) return launch_ssd_n<float, float, 128>(p, st);
    if (p.dstate == 64) return launch_ssd_n<float, float, 64>(p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mh
