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
//   1. ssd_chunk_state  grid (nchunks, H/HG, b): the chunk-local final state
//          S_k[p, n] = sum_{s in k} exp(sum_{s<tau in k} A dt_tau) dt_s x_s[p] B_s[n]
//      and the chunk's total log-decay T_k, walking the chunk forwards in
//      64-token segments with S in MFMA accumulators.
//   2. ssd_state_pass   elementwise over (b, h, P*N): H_0 = h0, H_{k+1} = e^{T_k} H_k + S_k.
//      Writes the *entering* state H_k over S_k and the final state.
//   3. ssd_chunk_scan   grid (nchunks, H/HG, b): walks the chunk in 64-token
//      segments with the running state H in MFMA accumulators.  With cs_t the
//      in-segment inclusive cumulative log-decay (cs_t <= 0, non-increasing):
//          y_t  = e^{cs_t} C_t H^T + sum_{s<=t} e^{cs_t - cs_s} (C_t . B_s) dt_s x_s + D x_t
//          H   <- e^{cs_end} H + sum_s e^{cs_end - cs_s} dt_s x_s B_s^T
//      Every factor of the state update is <= 1.  The intra-segment term is
//      factorised as e^{cs_t - m} * e^{m - cs_s} around the midpoint m of the
//      segment's log-decay range when that range is <= FACT_RANGE (both factors
//      within e^{+-30}), so the masked C B^T tile is shared by all heads of a
//      group; a segment with a wider range (very strong decay) takes an
//      exact per-element e^{cs_t - cs_s} path instead (wave-uniform branch).
// Work split: a workgroup owns HG heads of one group with two waves per head;
// wave w handles head w / 2 and the 32 state columns p of half w % 2, so each
// wave's state is N/32 accumulator tiles.  C B^T (three 32x32 tiles) and the
// B^T fragments are computed once per segment and shared by all waves.
// Transposes needed by the token-contracted MFMAs (B^T, x^T) are done on the
// MFMA unit itself: a row-loaded tile times an identity fragment lands in the
// accumulator layout that the next MFMA consumes.
// Memory: tiles of the next segment are fetched straight into a second LDS
// buffer (global_load_lds_dwordx4, no register staging) while the current one
// is computed.  Each wave owns the 32-column half of its head's x tile that it
// reads, so it stages its y columns in place of x and writes them to HBM one
// segment later, after the next segment's fetch has been issued: no wave ever
// waits for its own y stores.  LDS tiles are XOR-swizzled per row for
// conflict-free fragment reads; the chunk-state workspace is kept in MFMA
// fragment order (64 contiguous bytes per lane).
// bf16 I/O uses 32x32x16 bf16 MFMAs, fp32 I/O 32x32x2 fp32 MFMAs; accumulation is fp32.
#include "common.h"
#include "launch.h"

namespace mh {

constexpr int SEG = 64;              // tokens per segment
constexpr int HD = 64;               // headdim handled by these kernels
constexpr float FACT_RANGE = 60.f;   // max in-segment log-decay range of the factorised intra-segment path

// ------------------------------------------------------------------ helpers

__device__ __forceinline__ float process_dt(const SsdParams& p, float dt, int h) {
  if (p.dt_bias) dt += p.dt_bias[h];
  if (p.dt_softplus) dt = softplus_f(dt);
  if (p.has_dt_limit) dt = fminf(fmaxf(dt, p.dt_min), p.dt_max);
  return dt;
}

__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// ------------------------------------------------------------------ LDS tiles

// B / C tiles: SEG rows of W elements, unpadded, 16-byte chunks XOR-swizzled by
// row (chunk c of row r lives at chunk c ^ (r & MASK)) so the lanes of one LDS
// access phase, reading the same column of consecutive rows, hit distinct banks.
template <typename T, int W>
struct Tile {
  static constexpr int EPC = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  static constexpr int CPR = W / EPC;               // chunks per row (power of two)
  static constexpr int MASK = (CPR < 16 ? CPR : 16) - 1;
  static constexpr int RPB = 64 / CPR;              // rows per 1 KB block (one wave-wide direct load)
  static constexpr int NBLK = SEG / RPB;            // 1 KB blocks per tile
  __device__ static __forceinline__ int chunk(int r, int c) { return r * W + (c ^ (r & MASK)) * EPC; }
};

// One wave's half of a head's x tile: SEG token rows x 32 columns.  Rows of 64
// bytes (bf16) are swizzled with ((r >> 1) ^ (r >> 3)) & 3, which spreads the
// 16-byte reads of 16 consecutive rows over all banks whether the LDS serves
// 8 or 16 lanes of a 128-bit read per cycle; 128-byte rows (fp32) use r & 7.
template <typename T>
struct XHalf {
  static constexpr int W = 32;
  static constexpr int EPC = 16 / (int)sizeof(T);
  static constexpr int CPR = W / EPC;               // 4 (bf16) / 8 (fp32)
  static constexpr int RPB = 64 / CPR;              // 16 / 8 rows per 1 KB block
  static constexpr int NBLK = SEG / RPB;            // 4 / 8 blocks
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (CPR == 4) return ((r >> 1) ^ (r >> 3)) & 3;
    else return r & 7;
  }
  __device__ static __forceinline__ int chunk(int r, int c) { return r * W + (c ^ swz(r)) * EPC; }
};

// Direct global -> LDS fetch of 1 KB blocks [blk0, blk0 + nblk) of a swizzled
// B/C tile: lane i of the wave writes LDS bytes [16 i, 16 i + 16) of the block,
// so it fetches the logical chunk that the swizzle places there.  Rows past
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

// Direct fetch of a wave's x half tile (src points at column 0 of the half).
template <typename T>
__device__ __forceinline__ void fetch_xhalf(T* dst, const T* src, int64_t row_stride, int tok0, int last_tok,
                                            int lane) {
  using X = XHalf<T>;
  const int rr = lane / X::CPR, phys = lane % X::CPR;
#pragma unroll
  for (int blk = 0; blk < X::NBLK; ++blk) {
    const int r = blk * X::RPB + rr;
    const int c = phys ^ X::swz(r);
    const int tok = min(tok0 + r, last_tok);
    const T* g = src + (int64_t)tok * row_stride + c * X::EPC;
    T* d = dst + blk * (1024 / (int)sizeof(T));
    __builtin_amdgcn_global_load_lds((glb_void_t*)g, (lds_void_t*)d, 16, 0, 0);
  }
}

// Write the y rows [0, len) staged in a wave's x half tile to HBM (16-byte stores).
template <typename T>
__device__ __forceinline__ void store_yhalf(T* dst, int64_t row_stride, const T* tile, int len, int lane) {
  using X = XHalf<T>;
  uint4 v[X::NBLK];
#pragma unroll
  for (int i = 0; i < X::NBLK; ++i) {
    const int e = lane + 64 * i;
    v[i] = *reinterpret_cast<const uint4*>(tile + X::chunk(e / X::CPR, e % X::CPR));
  }
#pragma unroll
  for (int i = 0; i < X::NBLK; ++i) {
    const int e = lane + 64 * i;
    const int r = e / X::CPR, c = e % X::CPR;
    if (r < len) *reinterpret_cast<uint4*>(dst + (int64_t)r * row_stride + c * X::EPC) = v[i];
  }
  wait_lds();   // the staged rows have been read: the buffer may be refilled
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
template <typename TM, typename T>
__device__ __forceinline__ Frag<TM> xrow_frag(const T* tile, int r, int e0) {
  using X = XHalf<T>;
  Frag<TM> f;
  if constexpr (sizeof(T) == 2) {
    f.v = *reinterpret_cast<const bf16x8*>(tile + X::chunk(r, e0 / 8));
  } else {
    const f32x4 lo = *reinterpret_cast<const f32x4*>(tile + X::chunk(r, e0 / 4));
    const f32x4 hi = *reinterpret_cast<const f32x4*>(tile + X::chunk(r, e0 / 4 + 1));
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

// Values of a per-token array at the 8 tokens a KSET fragment covers (k-step c):
// tokens 16c+4*half+{0..3} and 16c+8+4*half+{0..3}, read as two float4.
__device__ __forceinline__ void kset_vals(const float* v, int c, int half, float (&s)[8]) {
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

// Transpose a 32x32 block of a row-major B tile through the MFMA unit:
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

// x^T of a wave's x half tile (lane = p, tokens on the k axis, KSET order) as
// two sets of 4 fragments: xa scaled per token by sa[], xb scaled by sb[].
template <typename TM, typename T, bool TWO>
__device__ __forceinline__ void xt_frags(const T* xtile, const float* sa, const float* sb, const Frag<TM> (&id)[2],
                                         int half, int l32, Frag<TM> (&xa)[4], Frag<TM> (&xb)[4]) {
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
      if constexpr (TWO) {
        kset_vals(sb, 2 * st + c, half, s);
#pragma unroll
        for (int j = 0; j < 8; ++j) xb[2 * st + c].set(j, xt[8 * c + j] * s[j]);
      }
    }
  }
}

// Shared per-segment MFMA work of a workgroup of NW waves: the three C B^T
// tiles (N/16 MFMAs each, k-reductions, one wave each) and the 2 * N/32 B^T
// blocks (2 MFMAs each), spread so the busiest wave does one C B^T tile.
template <int NW, int N, bool CB>
struct SharedWork {
  static constexpr int NBLK = 2 * (N / 32);
  static constexpr int NCB = CB ? 3 : 0;
  static constexpr int CBW = !CB ? 0 : (NW < 3 ? NW : 3);          // waves that own C B^T tiles
  static constexpr int BTW = (NW > CBW) ? NW - CBW : NW;          // waves that own B^T blocks
  static constexpr int BTP = (NBLK + BTW - 1) / BTW;
  static constexpr int CBPER = CB ? (3 + CBW - 1) / CBW : 0;
  __device__ static __forceinline__ int cb_tile(int w, int i) { return (w < CBW) ? w + i * CBW : 99; }
  __device__ static __forceinline__ int bt_block(int w, int i) {
    if (NW > CBW) return (w >= CBW) ? (w - CBW) + i * BTW : 99;
    return w + i * NW;
  }
};

// B^T A-operand fragments (row n, k = token via KSET) of one segment, in LDS.
template <typename TM, int N>
struct BtFrags {
  Frag<TM> f[N / 32][4][64];   // n-tile, k-step (16 tokens), lane
};

// Compute the B^T blocks a wave owns and store them as fragments.
template <typename T, typename TM, int N, int NW, bool CB>
__device__ __forceinline__ void bt_work(const T* Bs, BtFrags<TM, N>& bt, int w, const Frag<TM> (&id)[2], int half,
                                        int l32, int l) {
  using SW = SharedWork<NW, N, CB>;
#pragma unroll
  for (int i = 0; i < SW::BTP; ++i) {
    const int blk = SW::bt_block(w, i);
    if (blk < SW::NBLK) {
      const f32x16 acc = mfma_transpose<TM, T, N>(Bs, 32 * (blk & 1), 32 * (blk >> 1), id, half, l32);
      bt.f[blk >> 1][2 * (blk & 1)][l] = acc_to_frag<TM>(acc, 0);
      bt.f[blk >> 1][2 * (blk & 1) + 1][l] = acc_to_frag<TM>(acc, 1);
    }
  }
}

// Per-stage tiles.
template <typename T, int N, int HG>
struct ScanStage {
  T B[SEG * N];
  T C[SEG * N];
  T X[2 * HG][SEG * 32];      // per wave: its half of its head's x tile (y staged in place)
};
template <typename T, int N, int HG>
struct StateStage {
  T B[SEG * N];
  T X[2 * HG][SEG * 32];
};

template <typename T, typename TM, int N, int HG, int NBUF>
struct ScanSmem {
  ScanStage<T, N, HG> st[NBUF];
  BtFrags<TM, N> bt;
  Frag<TM> CB[3][2][64];      // masked (C B^T)^T tiles as B-operand fragments: tile, k-step, lane
  float sa[2 * HG][SEG];      // per wave: operand scale of the intra-segment term
  float sb[2 * HG][SEG];      // per wave: decay to the segment end, e^{cs_end - cs_s} (exact path)
  float cs[2 * HG][SEG];      // per wave: in-segment cumulative log-decay
  float dcol[HG][HD];         // D per column of each head
};
template <typename T, typename TM, int N, int HG, int NBUF>
struct StateSmem {
  StateStage<T, N, HG> st[NBUF];
  BtFrags<TM, N> bt;
  float sb[2 * HG][SEG];
};

// Tiles are double-buffered (the next segment fetched during this one's
// compute) where two buffers fit in the 160 KB of LDS, else single-buffered.
constexpr size_t LDS_BYTES = 160 * 1024;
template <typename T, typename TM, int N, int HG>
constexpr int scan_nbuf = sizeof(ScanSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1;
template <typename T, typename TM, int N, int HG>
constexpr int state_nbuf = sizeof(StateSmem<T, TM, N, HG, 2>) <= LDS_BYTES ? 2 : 1;

// Offset (floats) of state tile (nt, pt) element block of lane l in the fragment-native workspace order.
__device__ __forceinline__ int frag_off(int nt, int pt, int l) { return ((nt * 2 + pt) * 64 + l) * 16; }

// In-segment decay of one head (lane = token of the segment starting at pos,
// tokens at or past c1 have dt = 0): returns cs_t (inclusive cumulative log-decay).
__device__ __forceinline__ float seg_decay(const SsdParams& p, float dtraw, int h, float Ah, int t, int c1,
                                           float& dtv) {
  dtv = (t < c1) ? process_dt(p, dtraw, h) : 0.f;
  return wave_incl_scan(Ah * dtv);
}

// State read-out of one wave for one 32-token t-tile (rows tl of the C tile):
// Y^T[p][t] += sum_n H[p][n] C^T[n][t], H as A operand straight from the accumulators.
template <typename TM, typename T, int N>
__device__ __forceinline__ void readout(const f32x16 (&H)[N / 32], const T* Cs, int tl, int half, f32x16& Y) {
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt)
#pragma unroll
    for (int c = 0; c < 2; ++c) Y = mma(acc_to_frag<TM>(H[nt], c), kset_frag<TM, T, N>(Cs, tl, 32 * nt + 16 * c, half), Y);
}

// H[n][p] += sum_s B^T[n][s] xf[s][p] over the segment's 64 tokens.
template <typename TM, int N>
__device__ __forceinline__ void state_update(f32x16 (&H)[N / 32], const BtFrags<TM, N>& bt, const Frag<TM> (&xf)[4],
                                             int l) {
#pragma unroll
  for (int nt = 0; nt < N / 32; ++nt) {
    Frag<TM> btf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) btf[c] = bt.f[nt][c][l];
#pragma unroll
    for (int c = 0; c < 4; ++c) H[nt] = mma(btf[c], xf[c], H[nt]);
  }
}

// ------------------------------------------------------------------ kernel 1

template <typename T, typename TM, int N, int HG>
__global__ __launch_bounds__(128 * HG) void ssd_chunk_state_kernel(SsdParams p) {
  constexpr int NBUF = state_nbuf<T, TM, N, HG>;
  using SM = StateSmem<T, TM, N, HG, NBUF>;
  __shared__ SM sm;
  constexpr int NT = N / 32, NW = 2 * HG;
  using TB = Tile<T, N>;
  constexpr int BPW = (TB::NBLK + NW - 1) / NW;            // B blocks fetched per wave
  const int k = blockIdx.x, b = blockIdx.z;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int j = w >> 1, ph = w & 1;
  const int h = blockIdx.y * HG + j;
  const int g = h / (p.nheads / p.ngroups);
  const int c0 = k * p.chunk_len;
  const int c1 = min(p.seqlen, c0 + p.chunk_len);
  const int last = p.seqlen - 1;
  const float Ah = p.A[h];
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh + 32 * ph;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  const int b0 = w * BPW, nb = max(0, min(BPW, TB::NBLK - b0));
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);

  f32x16 S[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) S[nt] = zero16();
  float total = 0.f;

  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  float dtraw = (c0 + l < c1) ? dtg[(int64_t)(c0 + l) * p.dt_sl] : 0.f;
  fetch_tile<T, N>(sm.st[0].B, Bg, p.B_sl, c0, last, b0, nb, l);
  fetch_xhalf<T>(sm.st[0].X[w], xg, p.x_sl, c0, last, l);
  for (int si = 0; si < nseg; ++si) {
    int lq = l;
    asm volatile("" : "+v"(lq));
    const int ll = lq, halfq = lq >> 5, l32q = lq & 31;
    const int pos = c0 + si * SEG;
    const int cur = (NBUF == 2) ? (si & 1) : 0;
    auto& sg = sm.st[cur];
    if constexpr (NBUF == 1) {
      if (si > 0) {
        __syncthreads();                                   // every wave is done with the previous tiles
        fetch_tile<T, N>(sg.B, Bg, p.B_sl, pos, last, b0, nb, ll);
        fetch_xhalf<T>(sg.X[w], xg, p.x_sl, pos, last, ll);
      }
    }
    wait_vmem();
    __syncthreads();                                       // tiles of this segment are in LDS
    float dtn = 0.f;
    if constexpr (NBUF == 2) {
      if (si + 1 < nseg) {                                 // fetch the next segment into the other buffer
        auto& ng = sm.st[cur ^ 1];
        fetch_tile<T, N>(ng.B, Bg, p.B_sl, pos + SEG, last, b0, nb, ll);
        fetch_xhalf<T>(ng.X[w], xg, p.x_sl, pos + SEG, last, ll);
      }
    }
    if (si + 1 < nseg && pos + SEG + l < c1) dtn = dtg[(int64_t)(pos + SEG + l) * p.dt_sl];
    float dtv;
    const float cs = seg_decay(p, dtraw, h, Ah, pos + l, c1, dtv);
    const float cse = __shfl(cs, 63, 64);
    sm.sb[w][ll] = __expf(cse - cs) * dtv;
    bt_work<T, TM, N, NW, false>(sg.B, sm.bt, w, id, halfq, l32q, ll);
    __syncthreads();                                       // B^T fragments and scales visible
    Frag<TM> xw[4];
    xt_frags<TM, T, false>(sg.X[w], sm.sb[w], nullptr, id, halfq, l32q, xw, xw);
    const float e = __expf(cse);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) S[nt] *= e;
    state_update<TM, N>(S, sm.bt, xw, ll);
    total += cse;
    dtraw = dtn;
  }

  float* out = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    f32x4* o4 = reinterpret_cast<f32x4*>(out + frag_off(nt, ph, l));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      f32x4 v;
      v[0] = S[nt][4 * q]; v[1] = S[nt][4 * q + 1]; v[2] = S[nt][4 * q + 2]; v[3] = S[nt][4 * q + 3];
      o4[q] = v;
    }
  }
  if (l == 0 && ph == 0) p.chunk_decay[((int64_t)b * p.nheads + h) * p.nchunks + k] = total;
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
  constexpr int NT = N / 32, NW = 2 * HG;
  using SW = SharedWork<NW, N, true>;
  using TB = Tile<T, N>;
  using TX = XHalf<T>;
  constexpr int BPW = (TB::NBLK + NW - 1) / NW;            // B and C blocks fetched per wave
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
  const T* xg = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)h * p.x_sh + 32 * ph;
  const T* Bg = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)g * N;
  const T* Cg = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + (int64_t)g * N;
  const float* dtg = p.dt + (int64_t)b * p.dt_sb + h;
  T* yg = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + (int64_t)h * p.y_sh + 32 * ph;
  const int b0 = w * BPW, nb = max(0, min(BPW, TB::NBLK - b0));
  Frag<TM> id[2];
  id[0] = ident_frag<TM>(0, half, l32);
  id[1] = ident_frag<TM>(1, half, l32);
  if (ph == 0) sm.dcol[j][l] = p.D ? (p.D_per_channel ? p.D[h * HD + l] : p.D[h]) : 0.f;

  // Entering state H_k (fragment-native workspace order), columns of this wave's P-half.
  f32x16 H[NT];
  {
    const float* hk = p.chunk_states + (((int64_t)b * p.nchunks + k) * p.nheads + h) * (HD * N);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const f32x4* h4 = reinterpret_cast<const f32x4*>(hk + frag_off(nt, ph, l));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 v = h4[q];
        H[nt][4 * q] = v[0]; H[nt][4 * q + 1] = v[1]; H[nt][4 * q + 2] = v[2]; H[nt][4 * q + 3] = v[3];
      }
    }
  }

  const int nseg = (c1 - c0 + SEG - 1) / SEG;
  float dtraw = (c0 + l < c1) ? dtg[(int64_t)(c0 + l) * p.dt_sl] : 0.f;
  fetch_tile<T, N>(sm.st[0].B, Bg, p.B_sl, c0, last, b0, nb, l);
  fetch_tile<T, N>(sm.st[0].C, Cg, p.C_sl, c0, last, b0, nb, l);
  fetch_xhalf<T>(sm.st[0].X[w], xg, p.x_sl, c0, last, l);

  for (int si = 0; si < nseg; ++si) {
    // Lane-dependent LDS addresses are recomputed each segment (cheap VALU) instead of
    // being hoisted out of the loop, where they would all stay live and spill.
    int lq = l;
    asm volatile("" : "+v"(lq));
    const int ll = lq, halfq = lq >> 5, l32q = lq & 31;
    const int pos = c0 + si * SEG;
    const int cur = (NBUF == 2) ? (si & 1) : 0;
    auto& sg = sm.st[cur];
    T* xt = sg.X[w];
    if constexpr (NBUF == 1) {
      if (si > 0) {
        store_yhalf<T>(yg + (int64_t)(pos - SEG) * p.y_sl, p.y_sl, xt, SEG, ll);   // y of the previous segment
        __syncthreads();                                   // every wave is done with the previous tiles
        fetch_tile<T, N>(sg.B, Bg, p.B_sl, pos, last, b0, nb, ll);
        fetch_tile<T, N>(sg.C, Cg, p.C_sl, pos, last, b0, nb, ll);
        fetch_xhalf<T>(xt, xg, p.x_sl, pos, last, ll);
      }
    }
    wait_vmem();
    __syncthreads();                                       // tiles of this segment are in LDS
    float dtn = 0.f;
    if constexpr (NBUF == 2) {
      auto& og = sm.st[cur ^ 1];
      // y of the previous segment (staged in place of its x), then the next segment's fetch into the same buffer
      if (si > 0) store_yhalf<T>(yg + (int64_t)(pos - SEG) * p.y_sl, p.y_sl, og.X[w], SEG, ll);
      if (si + 1 < nseg) {
        fetch_tile<T, N>(og.B, Bg, p.B_sl, pos + SEG, last, b0, nb, ll);
        fetch_tile<T, N>(og.C, Cg, p.C_sl, pos + SEG, last, b0, nb, ll);
        fetch_xhalf<T>(og.X[w], xg, p.x_sl, pos + SEG, last, ll);
      }
    }
    if (si + 1 < nseg && pos + SEG + l < c1) dtn = dtg[(int64_t)(pos + SEG + l) * p.dt_sl];

    // ---- this head's in-segment decay (lane = token); the factorised path when the range is small
    const int len = min(SEG, c1 - pos);
    float dtv;
    const float cs = seg_decay(p, dtraw, h, Ah, pos + l, c1, dtv);
    const float cse = __shfl(cs, 63, 64);
    const bool fact = (-cse <= FACT_RANGE);               // wave-uniform
    const float m = fact ? 0.5f * cse : 0.f;
    sm.sa[w][ll] = (fact ? __expf(m - cs) : 1.f) * dtv;
    sm.sb[w][ll] = __expf(cse - cs);
    sm.cs[w][ll] = cs;

    // ---- shared: C B^T tiles (s-tile, t-tile) in {(0,0), (0,1), (1,1)} and B^T fragments
#pragma unroll
    for (int i = 0; i < SW::CBPER; ++i) {
      const int ti = SW::cb_tile(w, i);
      if (ti < 3) {
        const int st = (ti == 2) ? 1 : 0, tt = (ti == 0) ? 0 : 1;
        f32x16 acc = zero16();
#pragma unroll
        for (int c = 0; c < N / 16; ++c)
          acc = mma(row_frag<TM, T, N>(sg.B, 32 * st + l32q, 16 * c + 8 * halfq),
                    row_frag<TM, T, N>(sg.C, 32 * tt + l32q, 16 * c + 8 * halfq), acc);
        const int tl = 32 * tt + l32q;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int s = 32 * st + acc_row(halfq, r);
          if (!(s <= tl && s < len)) acc[r] = 0.f;
        }
        sm.CB[ti][0][ll] = acc_to_frag<TM>(acc, 0);
        sm.CB[ti][1][ll] = acc_to_frag<TM>(acc, 1);
      }
    }
    bt_work<T, TM, N, NW, true>(sg.B, sm.bt, w, id, halfq, l32q, ll);
    __syncthreads();                                       // C B^T, B^T fragments and scales visible

    // ---- per wave: head j, p-tile ph.  Y^T[p][t] = sum_n H[p][n] C^T[n][t] + sum_s xa^T[p][s] M^T[s][t],
    // one 32-token t-tile at a time (its y staged in place of x before the next).
    // Factorised path: H is carried at the segment midpoint, Hm = e^m H, with xa_s = e^{m - cs_s} dt_s x_s:
    //   y_t = e^{cs_t - m} (C_t Hm^T + sum_s M[t][s] xa_s),   H_end = e^{cse - m} (Hm + B^T xa).
    // Exact path (range above FACT_RANGE): xa_s = dt_s x_s, each masked C B^T entry decayed by
    // e^{cs_t - cs_s} (s <= t), the state term weighted by e^{cs_t}; H_end = e^{cse} H + B^T (e^{cse - cs} xa).
    Frag<TM> xa[4];
    xt_frags<TM, T, false>(xt, sm.sa[w], nullptr, id, halfq, l32q, xa, xa);
    if (fact) {
      const float em = __expf(m);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) H[nt] *= em;
    }
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tl = 32 * tt + l32q;
      const float cst = sm.cs[w][tl];
      f32x16 Y = zero16();
      readout<TM, T, N>(H, sg.C, tl, halfq, Y);
      float rsc = 1.f;
      if (fact) {
        if (tt == 0) {
          Y = mma(xa[0], sm.CB[0][0][ll], Y);
          Y = mma(xa[1], sm.CB[0][1][ll], Y);
        } else {
          Y = mma(xa[0], sm.CB[1][0][ll], Y);
          Y = mma(xa[1], sm.CB[1][1][ll], Y);
          Y = mma(xa[2], sm.CB[2][0][ll], Y);
          Y = mma(xa[3], sm.CB[2][1][ll], Y);
        }
        rsc = __expf(cst - m);
      } else {
        Y *= __expf(cst);
#pragma unroll
        for (int ti = tt; ti < 2 * tt + 1; ++ti) {         // tiles (s-tile, tt): tt = 0 -> {0}, tt = 1 -> {1, 2}
          const int st = (ti == 2) ? 1 : 0;
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            float css[8];
            kset_vals(sm.cs[w] + 32 * st, c, halfq, css);
            const Frag<TM> cb = sm.CB[ti][c][ll];
            Frag<TM> md;
#pragma unroll
            for (int e = 0; e < 8; ++e) md.set(e, cb.get(e) * __expf(fminf(cst - css[e], 0.f)));
            Y = mma(xa[2 * st + c], md, Y);
          }
        }
      }
      // y[t][p] = rsc Y + D x, staged in place of x
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int p0 = 8 * q + 4 * halfq;                // 4 consecutive columns of the half, inside one chunk
        T* xp = xt + TX::chunk(tl, (unsigned)p0 / TX::EPC) + ((unsigned)p0 % TX::EPC);
        const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.dcol[j][32 * ph + p0]);
        if constexpr (sizeof(T) == 2) {
          const bf16x4 xv = *reinterpret_cast<const bf16x4*>(xp);
          bf16x4 yv;
#pragma unroll
          for (int i = 0; i < 4; ++i) yv[i] = (bf16)(rsc * Y[4 * q + i] + d4[i] * (float)xv[i]);
          *reinterpret_cast<bf16x4*>(xp) = yv;
        } else {
          const f32x4 xv = *reinterpret_cast<const f32x4*>(xp);
          f32x4 yv;
#pragma unroll
          for (int i = 0; i < 4; ++i) yv[i] = rsc * Y[4 * q + i] + d4[i] * xv[i];
          *reinterpret_cast<f32x4*>(xp) = yv;
        }
      }
    }
    // ---- state update
    if (fact) {
      state_update<TM, N>(H, sm.bt, xa, ll);
      const float eo = __expf(cse - m);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) H[nt] *= eo;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {                        // xa <- e^{cse - cs_s} xa
        float f[8];
        kset_vals(sm.sb[w], c, halfq, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) xa[c].set(e, xa[c].get(e) * f[e]);
      }
      const float e = __expf(cse);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) H[nt] *= e;
      state_update<TM, N>(H, sm.bt, xa, ll);
    }
    dtraw = dtn;
  }
  // y of the last segment
  {
    const int si = nseg - 1;
    const int cur = (NBUF == 2) ? (si & 1) : 0;
    const int pos = c0 + si * SEG;
    store_yhalf<T>(yg + (int64_t)pos * p.y_sl, p.y_sl, sm.st[cur].X[w], c1 - pos, l);
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

template <typename T, typename TM, int N, int HG>
constexpr bool ssd_fits = sizeof(ScanSmem<T, TM, N, HG, 1>) <= LDS_BYTES && sizeof(StateSmem<T, TM, N, HG, 1>) <= LDS_BYTES;

template <typename T, typename TM, int N>
static hipError_t launch_ssd_n(const SsdParams& p, hipStream_t st) {
  switch (p.heads_per_wg) {
    case 4:
      if constexpr (ssd_fits<T, TM, N, 4>) return launch_ssd_t<T, TM, N, 4>(p, st);
      return hipErrorInvalidValue;
    case 2:
      if constexpr (ssd_fits<T, TM, N, 2>) return launch_ssd_t<T, TM, N, 2>(p, st);
      return hipErrorInvalidValue;
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
