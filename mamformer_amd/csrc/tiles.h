// LDS tile helpers shared by the chunked-scan kernels (gfx950): 64-row tiles
// fetched straight from HBM into LDS (global_load_lds), XOR-swizzled for
// conflict-free 16-byte fragment reads, MFMA operand fragments read out of
// them, and the identity-MFMA transpose.  Fragment conventions (KSET) are
// those of common.h.
#pragma once

#include "common.h"

namespace mh {

constexpr int SEG = 64;              // rows (tokens) per tile

// vmcnt(n) through the builtin (vmcnt n, expcnt 7, lgkmcnt 15), so the compiler's own wait tracking
// knows the counter state.  With only loads outstanding, they complete in issue order: vmcnt(n) waits for
// all but the n most recent (stores mixed in make the order unknown to the compiler, which then waits for 0).
template <int n>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(n >= 0 && n < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00);
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void wait_vmem() { wait_vmem_n<0>(); }
__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// ------------------------------------------------------------------ LDS tiles

// B / C tiles: SEG rows of W elements, unpadded, 16-byte chunks XOR-swizzled by
// row (chunk c of row r lives at chunk c ^ swz(r)) so the lanes of one LDS
// access phase hit distinct banks.  bf16 rows of 128 and 64 elements use swizzles
// under which both access shapes are conflict-free, whether the LDS has 32 or 64
// banks: 16-byte reads of one chunk in 8 or 16 consecutive rows, and the
// transposing reads (ds_read_b64_tr_b16), whose 16- or 32-lane phase reads 32 or
// 64 contiguous bytes of each of 4 consecutive rows (the rows' chunk sets then
// differ in bits 1-2 and in bits 2-3 of the chunk index).  Other tiles use r & MASK.
template <typename T, int W>
struct Tile {
  static constexpr int EPC = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  static constexpr int CPR = W / EPC;               // chunks per row (power of two)
  static constexpr int MASK = (CPR < 16 ? CPR : 16) - 1;
  static constexpr int RPB = 64 / CPR;              // rows per 1 KB block (one wave-wide direct load)
  static constexpr int NBLK = SEG / RPB;            // 1 KB blocks per tile
  __device__ static __forceinline__ int swz(int r) {
    if constexpr (sizeof(T) == 2 && W == 128)
      return (((r ^ (r >> 3)) & 1) << 3) | (((r >> 1) & 1) << 2) | ((r & 1) << 1) | ((r >> 2) & 1);
    else if constexpr (sizeof(T) == 2 && W == 64)
      return (((r >> 1) & 1) << 2) | (((r ^ (r >> 1) ^ (r >> 3)) & 1) << 1) | ((r >> 2) & 1);
    else
      return r & MASK;
  }
  __device__ static __forceinline__ int chunk(int r, int c) { return r * W + (c ^ swz(r)) * EPC; }
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

// 64-token tile of 32 16-bit columns (64-byte rows) whose 16-byte chunks are XOR-swizzled by (row >> 2) & 3;
// wider tiles are stored as consecutive such sub-tiles, one per 32-column slice.  With this layout the
// transposed reads (ds_read_b64_tr_b16: 8 rows x 64 bytes), row fragments (16 bytes of 32 rows) and
// 8-byte row accesses of 32 rows all spread over the LDS banks without conflicts beyond their minimum, and a
// lane's offset within a sub-tile depends only on its lane bits for every access pattern the kernels use.
struct Sub64 {
  static constexpr int W = 32;
  static constexpr int ELEMS = SEG * W;             // elements per sub-tile (4 KB of bf16)
  // element offset of (row r, column col) for col % 4 == 0, col < 32
  __host__ __device__ static constexpr int off(int r, int col) {
    return r * W + ((((col >> 3) ^ (r >> 2)) & 3) << 3) + (col & 7);
  }
};

// Direct global -> LDS load of `bytes` (16 or 4) per lane from a wave-uniform base plus a 32-bit lane
// offset (scalar-base addressing: no 64-bit per-lane address arithmetic).  Token strides are validated on
// the host so that a segment's span (SEG rows) stays below 2 GiB.
template <int bytes>
__device__ __forceinline__ void dma_lds(const void* base, uint32_t off, void* lds) {
  static_assert(bytes == 16 || bytes == 4, "direct-to-LDS load size");
  glb_void_t* g = (glb_void_t*)(reinterpret_cast<const char*>(base) + off);
  if constexpr (bytes == 16) __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 16, 0, 0);
  else __builtin_amdgcn_global_load_lds(g, (lds_void_t*)lds, 4, 0, 0);
}

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
  const T* base = src + (int64_t)tok0 * row_stride;       // wave-uniform
  const int rmax = last_tok - tok0;                        // >= 0; rows beyond it are clamped
  for (int q = 0; q < nblk; ++q) {
    const int blk = blk0 + q;
    const int r = blk * TL::RPB + rr;
    const int c = phys ^ TL::swz(r);
    const uint32_t off = (uint32_t)(min(r, rmax) * (int)row_stride + c * TL::EPC) * (uint32_t)sizeof(T);
    dma_lds<16>(base, off, dst + blk * (1024 / (int)sizeof(T)));
  }
}

// Direct fetch of 1 KB blocks [blk0, blk0 + nblk) of a Sub64-tiled bf16 tile of W columns (W / 32 sub-tiles of
// 4 blocks each): lane i of a block writes LDS bytes [16 i, 16 i + 16), i.e. row 16 (blk % 4) + i / 4 of
// sub-tile blk / 4 at physical chunk i % 4, so it fetches the logical chunk the swizzle places there.  Rows past
// `last_tok` re-read the last valid row.  The lane offsets are recomputed per call (lane_id_here).
__device__ __forceinline__ void fetch_sub64(bf16* dst, const bf16* src, int64_t row_stride, int tok0, int last_tok,
                                            int blk0, int nblk) {
  const bf16* base = src + (int64_t)tok0 * row_stride;   // wave-uniform
  const int rmax = last_tok - tok0;
  const int lane = lane_id_here();
  for (int q = 0; q < nblk; ++q) {
    const int blk = blk0 + q;
    const int r = 16 * (blk & 3) + (lane >> 2);
    const int c = (lane & 3) ^ ((r >> 2) & 3);
    const uint32_t off = (uint32_t)(min(r, rmax) * (int)row_stride + 32 * (blk >> 2) + 8 * c) * 2u;
    dma_lds<16>(base, off, dst + blk * 512);
  }
}

// Direct fetch of a wave's x half tile (src points at column 0 of the half).
template <typename T>
__device__ __forceinline__ void fetch_xhalf(T* dst, const T* src, int64_t row_stride, int tok0, int last_tok,
                                            int lane) {
  using X = XHalf<T>;
  const int rr = lane / X::CPR, phys = lane % X::CPR;
  const T* base = src + (int64_t)tok0 * row_stride;
  const int rmax = last_tok - tok0;
#pragma unroll
  for (int blk = 0; blk < X::NBLK; ++blk) {
    const int r = blk * X::RPB + rr;
    const int c = phys ^ X::swz(r);
    const uint32_t off = (uint32_t)(min(r, rmax) * (int)row_stride + c * X::EPC) * (uint32_t)sizeof(T);
    dma_lds<16>(base, off, dst + blk * (1024 / (int)sizeof(T)));
  }
}

// Direct fetch of the raw dt of 64 tokens (lane = token, rows past the end clamped) into LDS.
__device__ __forceinline__ void fetch_dt(float* dst, const float* src, int64_t stride, int tok0, int last_tok,
                                         int lane) {
  const float* base = src + (int64_t)tok0 * stride;
  dma_lds<4>(base, (uint32_t)(min(lane, last_tok - tok0) * (int)stride) * 4u, dst);
}

// Direct copy of nb contiguous 1 KB blocks starting at block b0 (precomputed fragments).
__device__ __forceinline__ void fetch_blocks(char* dst, const char* src, int b0, int nb, int lane) {
  for (int q = 0; q < nb; ++q) dma_lds<16>(src + (b0 + q) * 1024, 16u * lane, dst + (b0 + q) * 1024);
}

// y rows staged in a wave's x half tile: lane-held 16-byte chunks (read), then written to HBM.
template <typename T>
__device__ __forceinline__ void load_yhalf(const T* tile, int lane, uint4 (&v)[XHalf<T>::NBLK]) {
  using X = XHalf<T>;
#pragma unroll
  for (int i = 0; i < X::NBLK; ++i) {
    const int e = lane + 64 * i;
    v[i] = *reinterpret_cast<const uint4*>(tile + X::chunk(e / X::CPR, e % X::CPR));
  }
}
// All SEG rows (a full segment): exactly NBLK store instructions per wave, whatever the lane.
template <typename T>
__device__ __forceinline__ void store_yhalf_full(T* dst, int64_t row_stride, const uint4 (&v)[XHalf<T>::NBLK],
                                                 int lane) {
  using X = XHalf<T>;
#pragma unroll
  for (int i = 0; i < X::NBLK; ++i) {
    const int e = lane + 64 * i;
    *reinterpret_cast<uint4*>(dst + (int64_t)(e / X::CPR) * row_stride + (e % X::CPR) * X::EPC) = v[i];
  }
}
// Output gate on the staged y chunks: y <- y * silu(z), z chunks in the same lane order.
template <typename T>
__device__ __forceinline__ void gate_chunks(uint4 (&v)[XHalf<T>::NBLK], const uint4 (&z)[XHalf<T>::NBLK]) {
#pragma unroll
  for (int i = 0; i < XHalf<T>::NBLK; ++i) {
    if constexpr (sizeof(T) == 2) {
      bf16x8 y = __builtin_bit_cast(bf16x8, v[i]);
      const bf16x8 g = __builtin_bit_cast(bf16x8, z[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = (bf16)((float)y[j] * silu_f((float)g[j]));
      v[i] = __builtin_bit_cast(uint4, y);
    } else {
      f32x4 y = __builtin_bit_cast(f32x4, v[i]);
      const f32x4 g = __builtin_bit_cast(f32x4, z[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] *= silu_f(g[j]);
      v[i] = __builtin_bit_cast(uint4, y);
    }
  }
}

// Gate chunks z of a wave's 32-column half, rows [0, SEG) of src (rows past rmax re-read row rmax), in
// the lane order of load_yhalf.
template <typename T>
__device__ __forceinline__ void load_zhalf(const T* src, int64_t row_stride, int rmax, int lane,
                                           uint4 (&v)[XHalf<T>::NBLK]) {
  using X = XHalf<T>;
#pragma unroll
  for (int i = 0; i < X::NBLK; ++i) {
    const int e = lane + 64 * i;
    v[i] = *reinterpret_cast<const uint4*>(src + (int64_t)min(e / X::CPR, rmax) * row_stride + (e % X::CPR) * X::EPC);
  }
}

// Rows [0, len) only; with `gate`, y <- y * silu(z) on the z chunks loaded with load_zhalf.
template <typename T>
__device__ __forceinline__ void store_yhalf(T* dst, int64_t row_stride, const T* tile, int len, int lane, bool gate,
                                            const uint4 (&zv)[XHalf<T>::NBLK]) {
  using X = XHalf<T>;
  uint4 v[X::NBLK];
  load_yhalf<T>(tile, lane, v);
  if (gate) gate_chunks<T>(v, zv);
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
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// Fragment with k-values M[k0 + KSET(half, j)][c0 + lane % 32] (k runs down a column of a row-major bf16 LDS
// tile of the given pitch), by two transposing reads (ds_read_b64_tr_b16: within each 16-lane group, lanes
// 4r..4r+3 name 4 consecutive elements each of row r = 0..3, 16 in all, and lane i of the group receives element
// i of the four rows): rows k0 + 4 half + 0..3, then 8 further down.  Rows 8-byte aligned (pitch % 4 == 0),
// c0 % 32 == 0.
__device__ __forceinline__ Frag<bf16> col_frag_tr(const bf16* M, int pitch, int c0, int k0) {
  const int l = threadIdx.x & 63, half = l >> 5, i = l & 15;
  const bf16* p = M + (k0 + 4 * half + (i >> 2)) * pitch + c0 + 16 * ((l >> 4) & 1) + 4 * (i & 3);
  const i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
  const i16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 8 * pitch));
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
  return f;
}

// The same fragment from a swizzled Tile<bf16, W> (k = row, c0 % 32 == 0): each lane's 8-byte piece lies inside
// one 16-byte chunk, whose place in its row the swizzle gives.
template <int W>
__device__ __forceinline__ Frag<bf16> col_frag_tr_tile(const bf16* M, int c0, int k0) {
  using TL = Tile<bf16, W>;
  const int l = threadIdx.x & 63, half = l >> 5, i = l & 15;
  const int r = k0 + 4 * half + (i >> 2), col = c0 + 16 * ((l >> 4) & 1) + 4 * (i & 3);
  const bf16* p0 = M + TL::chunk(r, col >> 3) + (col & 7);
  const bf16* p1 = M + TL::chunk(r + 8, col >> 3) + (col & 7);
  const i16x4_t a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p0));
  const i16x4_t b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p1));
  Frag<bf16> f;
  f.v = __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
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

}  // namespace mh
