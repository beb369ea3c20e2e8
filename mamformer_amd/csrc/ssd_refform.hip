// The reference's own selective scan (mamformer/layers/mamba2.py:70-130) for gfx950: a decay rate per state
// column and a step size per channel,
//     h_t[c, n] = exp(A_n dt_t[c]) h_{t-1}[c, n] + dt_t[c] x_t[c] B_t[n],   y_t[c] = sum_n C_t[n] h_t[c, n] + D_c x_t[c]
// with A_n = -exp(clamp(A_log_n, -5, 5)) formed by the caller.  The decay differs per (channel, state), so the
// recurrence has no matrix-unit factorisation (the per-head SSD form does): every (token, channel, state) costs
// one exponential and a few fused multiply-adds, and the kernels are bound by that VALU work.
//
// rf_scan_kernel, one workgroup per (batch, block of channels), walking the whole sequence:
//   LPC = 32 lanes per channel (16 for N = 16), each owning N / 32 consecutive states, so the sum over states
//   that forms y runs on the DPP crossbar (quad permutes, the row mirrors, then the row-15 broadcast that adds
//   the two rows of a channel); a wave holds 2 channels, a workgroup of 4 waves 8.  Blocks of TB tokens of B, C
//   (fp32), dt, x and the gate are staged in LDS (two stages; the next block's rows are loaded into registers
//   while the current block computes, and each token's LDS values are read one token ahead), y is collected per
//   block in LDS and stored as rows of the workgroup's channels.
// rf_hs_kernel (h_states, the per-token mean of the state over all channels, mamba2.py:114-116):
//   lane = channel (256 channels per workgroup), a workgroup per (batch, channel block, group of 4 states), so
//   that the sum over channels is a reduce-scatter inside the wave (v_permlane32_swap, v_permlane16_swap, then the
//   DPP row sums) plus a sum over the 4 waves; the per-block sums go to a workspace and rf_hs_reduce_kernel adds
//   them in a fixed order (deterministic).
#include "common.h"
#include "launch.h"
#include "ssd_shared.h"

namespace mh {

namespace {

constexpr int RF_NT = 256;           // threads per workgroup (both kernels)
constexpr int HS_CPB = 256;          // channels per workgroup of h_states
constexpr int HS_NS = 4;             // states per thread of h_states
constexpr int HS_TB = 16;            // tokens per block of h_states
constexpr float LOG2E = 1.4426950408889634f;

// Lanes per channel of the scan, states per lane, channels per workgroup, tokens per LDS block.
template <int N> constexpr int rf_lpc() { return N >= 32 ? 32 : 16; }
template <int N> constexpr int rf_ns() { return N / rf_lpc<N>(); }
template <int N> constexpr int rf_cpb() { return 4 * (64 / rf_lpc<N>()); }
template <int N> constexpr int rf_tb() { return N <= 128 ? 32 : 16; }
// Tokens per piece of the backward (the checkpoint spacing): the per-token states and decays of a piece are held in
// registers, RK * NS of each per lane.
template <int N> constexpr int rf_rk() { return rf_ns<N>() <= 4 ? 16 : 8; }

// Per-lane token prologue: dt <- clamp(softplus?(dt + bias), dt_min, dt_max).
__device__ __forceinline__ float rf_dt(const RfParams& p, float raw, float bias) {
  float d = raw + bias;
  if (p.dt_softplus) d = softplus_f(d);
  if (p.has_dt_limit) d = fminf(fmaxf(d, p.dt_min), p.dt_max);
  return d;
}

// Sum over each 16-lane row, in every lane of the row: quad permutes, then the half-row and row mirrors.
__device__ __forceinline__ float row_sum16(float v) {
  v += dppf<0xB1>(v);      // quad_perm 1,0,3,2
  v += dppf<0x4E>(v);      // quad_perm 2,3,0,1
  v += dppf<0x141>(v);     // row_half_mirror
  v += dppf<0x140>(v);     // row_mirror
  return v;
}

// Lane-crossing moves within 16-lane rows (DPP): the value of lane l ^ 8, ^ 4, ^ 2, ^ 1 of the same row.
__device__ __forceinline__ float xor8(float v) { return dppf<0x128>(v); }       // row_ror:8
__device__ __forceinline__ float xor4(float v) {
  // lanes 4-7 and 12-15 (banks 1, 3) read lane l - 4, lanes 0-3 and 8-11 (banks 0, 2) lane l + 4
  const int a = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xa, false);   // row_shr:4
  return __int_as_float(__builtin_amdgcn_update_dpp(a, __float_as_int(v), 0x104, 0xf, 0x5, false));   // row_shl:4
}
__device__ __forceinline__ float xor2(float v) { return dppf<0x4E>(v); }        // quad_perm 2,3,0,1
__device__ __forceinline__ float xor1(float v) { return dppf<0xB1>(v); }        // quad_perm 1,0,3,2

// One step of the reduce-scatter below: the lanes with lane bit M set keep the upper half of their first K
// values and hand the lower half to the partner l ^ M, which keeps its lower half.
template <int M, int K, int NV>
__device__ __forceinline__ void rf_rs_step(float (&v)[NV], int l) {
  const bool up = (l & M) != 0;
#pragma unroll
  for (int k = 0; k < K / 2; ++k) {
    const float keep = up ? v[k + K / 2] : v[k], send = up ? v[k] : v[k + K / 2];
    float r;
    if constexpr (M == 8) r = xor8(send);
    else if constexpr (M == 4) r = xor4(send);
    else if constexpr (M == 2) r = xor2(send);
    else r = xor1(send);
    v[k] = keep + r;
  }
}

// Sums of v[t] (t < 32) over the 32 lanes of a channel (lanes 32 c .. 32 c + 31, two 16-lane rows), lane g of
// the channel ending with the sum for t = g: one exchange-and-add per value pair and step, 31 for 32 tokens,
// where a separate row sum per token took five dependent DPP additions.
__device__ __forceinline__ float rf_reduce_scatter32(float (&v)[32], int l) {
  // lane bit 16: v_permlane16_swap trades the odd rows of its first operand with the even rows of its second,
  // so row 0 of the channel ends with v[k] of both rows and row 1 with v[k + 16] of both
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  rf_rs_step<8, 16>(v, l);
  rf_rs_step<4, 8>(v, l);
  rf_rs_step<2, 4>(v, l);
  rf_rs_step<1, 2>(v, l);
  return v[0];
}

// 16 values over the 32 lanes of a channel: lanes 2 m and 2 m + 1 of the channel end with the sum of v[m].
__device__ __forceinline__ float rf_reduce_scatter32_16(float (&v)[16], int l) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 8]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  rf_rs_step<8, 8>(v, l);
  rf_rs_step<4, 4>(v, l);
  rf_rs_step<2, 2>(v, l);
  return v[0] + xor1(v[0]);
}

// 32 values over all 64 lanes of the wave: lanes 2 m and 2 m + 1 end with the sum of v[m].
__device__ __forceinline__ float rf_reduce_scatter64_32(float (&v)[32], int l) {
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 8]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  rf_rs_step<8, 8>(v, l);
  rf_rs_step<4, 4>(v, l);
  rf_rs_step<2, 2>(v, l);
  return v[0] + xor1(v[0]);
}

// The same over all 64 lanes of the wave: lane l ends with the sum of v[l] (v_permlane32_swap first).
__device__ __forceinline__ float rf_reduce_scatter64(float (&v)[64], int l) {
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 32]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[k]), __float_as_uint(v[k + 16]), false, false);
    v[k] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  rf_rs_step<8, 16>(v, l);
  rf_rs_step<4, 8>(v, l);
  rf_rs_step<2, 4>(v, l);
  rf_rs_step<1, 2>(v, l);
  return v[0];
}

// 8 consecutive elements of a row: load, convert to fp32, pack from fp32, store.
template <typename T> struct Row8;
template <> struct Row8<bf16> {
  uint4 v;
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void set(const float* s) {
    bf16x8 b;
#pragma unroll
    for (int j = 0; j < 8; ++j) b[j] = (bf16)s[j];
    v = __builtin_bit_cast(uint4, b);
  }
  __device__ __forceinline__ void store(bf16* d) const { *reinterpret_cast<uint4*>(d) = v; }
  __device__ __forceinline__ void store_f32(float* d) const {
    const bf16x8 b = __builtin_bit_cast(bf16x8, v);
    reinterpret_cast<float4*>(d)[0] = float4{(float)b[0], (float)b[1], (float)b[2], (float)b[3]};
    reinterpret_cast<float4*>(d)[1] = float4{(float)b[4], (float)b[5], (float)b[6], (float)b[7]};
  }
};
template <> struct Row8<float> {
  f32x4 a, b;                  // (vector types that stay in registers: a struct of float4 went to scratch)
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const f32x4*>(p)[0];
    b = reinterpret_cast<const f32x4*>(p)[1];
  }
  __device__ __forceinline__ void set(const float* s) {
    a = f32x4{s[0], s[1], s[2], s[3]};
    b = f32x4{s[4], s[5], s[6], s[7]};
  }
  __device__ __forceinline__ void store(float* d) const {
    reinterpret_cast<f32x4*>(d)[0] = a;
    reinterpret_cast<f32x4*>(d)[1] = b;
  }
  __device__ __forceinline__ void store_f32(float* d) const { store(d); }
};

template <int N, int TB, int CPB>
struct __align__(16) RfStage {
  // 16-byte aligned rows, so that a lane's 4 states of B and C are one 16-byte LDS read at an immediate offset
  __align__(16) float B[TB][N];
  __align__(16) float C[TB][N];
  float dt[TB][CPB];        // processed dt (0 past the sequence)
  float x[TB][CPB];         // x (0 past the sequence)
  float z[TB][CPB];         // gate (GATE only)
};
template <int N, int TB, int CPB>
struct RfSmem {
  RfStage<N, TB, CPB> st[2];
  float y[2][TB][CPB];
};

// The rows of one token block held in registers between its load and its LDS store: thread i owns the 8-element
// pieces i, i + 256, .. of B and of C (TB rows of N), and, for i < TB * CPB / 4, one 4-element piece of dt, x, z.
template <typename T, int N, int TB, int CPB>
struct RfRegs {
  static constexpr int NP = TB * N / 8;                     // 8-element pieces of B (and of C) per block
  static constexpr int PB = (NP + RF_NT - 1) / RF_NT;      // per thread
  static constexpr int NQ = TB * CPB / 4;                  // 4-element pieces of dt (x, z) per block
  Row8<T> b[PB], c[PB];
  float4 dt;                   // raw dt; processed (bias, softplus, clamp, 0 past the end) by rf_store
  T xv[4], zv[4];              // raw x and gate
};

// Workgroup -> (batch, channel block): runs of 4 consecutive blocks go to the same XCD (workgroups are dealt to
// the 8 XCDs round-robin), so the x, y and z lines they share are read or written through one L2.
__device__ __forceinline__ void rf_block(int nblk, int nper, int& b, int& cb) {
  const int i = blockIdx.x;
  int j = i;
  if ((nblk & 31) == 0) j = 4 * ((i & 7) + 8 * (i >> 5)) + ((i >> 3) & 3);
  b = j / nper;
  cb = j % nper;
}

// Workgroup index of the channel-major walks (rf_hs_kernel, rf_bwd_state_kernel: (batch, channel block, state
// group), state group fastest), remapped so that each XCD runs a contiguous range of them: the state groups of a
// channel block then read its rows of dt, x and dy through one L2 (workgroups are dealt to the 8 XCDs
// round-robin; dealt as they come, each row was fetched by all eight).
__device__ __forceinline__ int rf_xcd_block() {
  const int i = blockIdx.x, n = gridDim.x;
  if (n % 8 != 0) return i;
  return (i & 7) * (n >> 3) + (i >> 3);
}

// Loads only (every one unconditional at a clamped row), so that they stay in flight while the current block
// computes: the values are converted, masked and stored to LDS by rf_store a block later.
template <typename T, int N, int TB, int CPB, bool GATE>
__device__ __forceinline__ void rf_load(const RfParams& p, RfRegs<T, N, TB, CPB>& r, int b, int c0, int t0) {
  using R = RfRegs<T, N, TB, CPB>;
  const int tid = threadIdx.x;
  const int last = p.seqlen - 1;
  const T* Bp = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb;
  const T* Cp = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb;
#pragma unroll
  for (int q = 0; q < R::PB; ++q) {
    const int e = min(tid + q * RF_NT, R::NP - 1);        // piece: row e / (N / 8), columns 8 (e % (N / 8))
    const int row = min(t0 + e / (N / 8), last), col = 8 * (e % (N / 8));
    r.b[q].load(Bp + (int64_t)row * p.B_sl + col);
    r.c[q].load(Cp + (int64_t)row * p.C_sl + col);
  }
  if (tid < R::NQ) {
    const int row = t0 + tid / (CPB / 4), col = 4 * (tid % (CPB / 4));
    const int rr = min(row, last);
    r.dt = *reinterpret_cast<const float4*>(p.dt + (int64_t)b * p.dt_sb + (int64_t)rr * p.dt_sl + c0 + col);
    const T* xp = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + (int64_t)rr * p.x_sl + c0 + col;
#pragma unroll
    for (int j = 0; j < 4; ++j) r.xv[j] = xp[j];
    if constexpr (GATE) {
      const T* zp = reinterpret_cast<const T*>(p.z) + (int64_t)b * p.z_sb + (int64_t)rr * p.z_sl + c0 + col;
#pragma unroll
      for (int j = 0; j < 4; ++j) r.zv[j] = zp[j];
    }
  }
}

// The block at t0 into LDS: B and C as fp32; dt processed with the thread's 4 channels' bias (bias4), dt and x 0
// past the end of the sequence.
template <typename T, int N, int TB, int CPB, bool GATE>
__device__ __forceinline__ void rf_store(const RfParams& p, const RfRegs<T, N, TB, CPB>& r, RfStage<N, TB, CPB>& s,
                                         int t0, const float4& bias4) {
  using R = RfRegs<T, N, TB, CPB>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int q = 0; q < R::PB; ++q) {
    const int e = tid + q * RF_NT;
    if (R::NP % RF_NT != 0 && e >= R::NP) break;
    r.b[q].store_f32(&s.B[e / (N / 8)][8 * (e % (N / 8))]);
    r.c[q].store_f32(&s.C[e / (N / 8)][8 * (e % (N / 8))]);
  }
  if (tid < R::NQ) {
    const int row = tid / (CPB / 4), col = 4 * (tid % (CPB / 4));
    const float in = t0 + row < p.seqlen ? 1.f : 0.f;
    *reinterpret_cast<float4*>(&s.dt[row][col]) =
        float4{rf_dt(p, r.dt.x, bias4.x) * in, rf_dt(p, r.dt.y, bias4.y) * in, rf_dt(p, r.dt.z, bias4.z) * in,
               rf_dt(p, r.dt.w, bias4.w) * in};
    *reinterpret_cast<float4*>(&s.x[row][col]) =
        float4{to_f32(r.xv[0]) * in, to_f32(r.xv[1]) * in, to_f32(r.xv[2]) * in, to_f32(r.xv[3]) * in};
    if constexpr (GATE)
      *reinterpret_cast<float4*>(&s.z[row][col]) =
          float4{to_f32(r.zv[0]), to_f32(r.zv[1]), to_f32(r.zv[2]), to_f32(r.zv[3])};
  }
}

// One token's operands, read from LDS a token ahead of their use.
template <int NS>
struct RfTok {
  float dt, x, b[NS], c[NS];
};
template <int N, int TB, int CPB, int NS>
__device__ __forceinline__ void rf_tok(const RfStage<N, TB, CPB>& s, int t, int cl, int n0, RfTok<NS>& o) {
  o.dt = s.dt[t][cl];
  o.x = s.x[t][cl];
  if constexpr (NS % 4 == 0) {
#pragma unroll
    for (int q = 0; q < NS; q += 4) {
      const float4 b4 = *reinterpret_cast<const float4*>(&s.B[t][n0 + q]);
      const float4 c4 = *reinterpret_cast<const float4*>(&s.C[t][n0 + q]);
      o.b[q] = b4.x; o.b[q + 1] = b4.y; o.b[q + 2] = b4.z; o.b[q + 3] = b4.w;
      o.c[q] = c4.x; o.c[q + 1] = c4.y; o.c[q + 2] = c4.z; o.c[q + 3] = c4.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < NS; ++q) {
      o.b[q] = s.B[t][n0 + q];
      o.c[q] = s.C[t][n0 + q];
    }
  }
}

// CKPT: the checkpoint pass of the backward, which writes the state entering every piece of rf_rk<N>() tokens
// (p.ckpt) and no y.
template <typename T, int N, bool GATE, bool CKPT = false>
__global__ __launch_bounds__(RF_NT) void rf_scan_kernel(RfParams p) {
  constexpr int TB = rf_tb<N>(), LPC = rf_lpc<N>(), NS = rf_ns<N>(), CPB = rf_cpb<N>();
  __shared__ RfSmem<N, TB, CPB> sm;
  const int nper = p.d_inner / CPB;
  int b, cb;
  rf_block(p.batch * nper, nper, b, cb);
  const int c0 = cb * CPB;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int cl = (64 / LPC) * w + lane / LPC, g = lane % LPC;   // channel within the workgroup, its state group
  const int c = c0 + cl;
  const int n0 = g * NS;
  // the lane that ends up with the channel's y: after the row sums (and, for two rows, the row-15 broadcast
  // into the channel's second row) every lane of the last row holds it; take the row's last lane
  const bool ylane = g == LPC - 1;
  float k2[NS], h[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    k2[s] = p.A[n0 + s] * LOG2E;                           // exp(A dt) = 2^(A log2(e) dt)
    h[s] = p.init_state ? p.init_state[((int64_t)b * p.d_inner + c) * N + n0 + s] : 0.f;
  }
  const float Dc = p.D ? (p.D_per_channel ? p.D[c] : p.D[c / p.headdim]) : 0.f;
  const int nblk = (p.seqlen + TB - 1) / TB;
  RfRegs<T, N, TB, CPB> r;
  float4 bias4 = {0.f, 0.f, 0.f, 0.f};      // this thread's 4 channels of dt_bias (the same rows every block)
  if (p.dt_bias && tid < RfRegs<T, N, TB, CPB>::NQ)
    bias4 = *reinterpret_cast<const float4*>(p.dt_bias + c0 + 4 * (tid % (CPB / 4)));
  if (nblk > 0) {
    rf_load<T, N, TB, CPB, GATE>(p, r, b, c0, 0);
    rf_store<T, N, TB, CPB, GATE>(p, r, sm.st[0], 0, bias4);
  }
  if (nblk > 1) rf_load<T, N, TB, CPB, GATE>(p, r, b, c0, TB);
  __syncthreads();
  T* yb = reinterpret_cast<T*>(p.y) + (int64_t)b * p.y_sb + c0;
  for (int k = 0; k < nblk; ++k) {
    const RfStage<N, TB, CPB>& s = sm.st[k & 1];
    float (*ys)[CPB] = sm.y[k & 1];
    if constexpr (TB == LPC && LPC == 32) {
      // the block's 32 tokens unrolled: every token's y is left as one partial per lane, and a reduce-scatter
      // over the channel's 32 lanes after the block hands lane g the sum for token g (CKPT: no y; the state
      // entering every piece is stored)
      float yacc[32];
#pragma unroll
      for (int t = 0; t < TB; ++t) {
        if constexpr (CKPT) {
          constexpr int RK = rf_rk<N>();                   // divides TB: a piece starts where t % RK == 0
          const int tt = k * TB + t;
          if (t % RK == 0 && tt < p.seqlen) {
            const int nsb = (p.seqlen + RK - 1) / RK;
            float* o = p.ckpt + (((int64_t)b * nsb + tt / RK) * p.d_inner + c) * N + n0;
#pragma unroll
            for (int s2 = 0; s2 < NS; ++s2) o[s2] = h[s2];
          }
        }
        RfTok<NS> o;
        rf_tok<N, TB, CPB, NS>(s, t, cl, n0, o);
        const float u = o.dt * o.x;
        float yp = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < NS; ++s2) {
          const float a = __builtin_amdgcn_exp2f(o.dt * k2[s2]);
          h[s2] = fmaf(a, h[s2], u * o.b[s2]);
          yp = fmaf(o.c[s2], h[s2], yp);
        }
        yacc[t] = yp;
      }
      if constexpr (!CKPT) {
        float yv = rf_reduce_scatter32(yacc, lane);
        yv += Dc * s.x[g][cl];
        if constexpr (GATE) yv *= silu_f(s.z[g][cl]);
        ys[g][cl] = yv;
      }
    } else {
    RfTok<NS> cur, nxt;
    rf_tok<N, TB, CPB, NS>(s, 0, cl, n0, cur);
#pragma unroll 2
    for (int t = 0; t < TB; ++t) {
      if (t + 1 < TB) rf_tok<N, TB, CPB, NS>(s, t + 1, cl, n0, nxt);
      if constexpr (CKPT) {
        constexpr int RK = rf_rk<N>();                     // divides TB: a piece starts where t % RK == 0
        const int tt = k * TB + t;
        if (t % RK == 0 && tt < p.seqlen) {
          const int nsb = (p.seqlen + RK - 1) / RK;
          float* o = p.ckpt + (((int64_t)b * nsb + tt / RK) * p.d_inner + c) * N + n0;
#pragma unroll
          for (int s2 = 0; s2 < NS; ++s2) o[s2] = h[s2];
        }
      }
      const float u = cur.dt * cur.x;
      float yp = 0.f;
#pragma unroll
      for (int s2 = 0; s2 < NS; ++s2) {
        const float a = __builtin_amdgcn_exp2f(cur.dt * k2[s2]);
        h[s2] = fmaf(a, h[s2], u * cur.b[s2]);
        yp = fmaf(cur.c[s2], h[s2], yp);
      }
      if constexpr (!CKPT) {
        yp = row_sum16(yp);
        if constexpr (LPC == 32) yp += dppf<0x142, 0xa>(yp);   // row_bcast:15 -> rows 1, 3: both rows of a channel
        if (ylane) {
          float yv = yp + Dc * cur.x;
          if constexpr (GATE) yv *= silu_f(s.z[t][cl]);
          ys[t][cl] = yv;
        }
      }
      cur = nxt;
    }
    }
    if (k + 1 < nblk) rf_store<T, N, TB, CPB, GATE>(p, r, sm.st[(k + 1) & 1], (k + 1) * TB, bias4);
    if (k + 2 < nblk) rf_load<T, N, TB, CPB, GATE>(p, r, b, c0, (k + 2) * TB);
    __syncthreads();
    // y rows of this block: CPB channels = CPB / 8 pieces of 8 per token
    if (!CKPT && tid < TB * (CPB / 8)) {
      const int t = tid / (CPB / 8), piece = tid % (CPB / 8);
      const int row = k * TB + t;
      if (row < p.seqlen) {
        Row8<T> o;
        o.set(&ys[t][8 * piece]);
        o.store(yb + (int64_t)row * p.y_sl + 8 * piece);
      }
    }
  }
  if (!CKPT && p.final_state) {
    float* fo = p.final_state + ((int64_t)b * p.d_inner + c) * N + n0;
#pragma unroll
    for (int q = 0; q < NS; ++q) fo[q] = h[q];
  }
}

// h_states: sums over the workgroup's 256 channels of every state of group gs (4 states), per token, into
// part[(b * ncb + cblk) * L + t][N]; channels past d_inner stay zero.
template <typename T, int N>
__global__ __launch_bounds__(RF_NT) void rf_hs_kernel(RfParams p) {
  __shared__ float red[4][HS_TB][HS_NS];
  __shared__ float4 sB[2][HS_TB];                          // the group's 4 states of B per token
  const int ncb = (p.d_inner + HS_CPB - 1) / HS_CPB, ngs = N / HS_NS;
  const int i = rf_xcd_block();
  const int gs = i % ngs, cblk = (i / ngs) % ncb, b = i / (ngs * ncb);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = cblk * HS_CPB + tid;
  const bool on = c < p.d_inner;
  const int cc = on ? c : p.d_inner - 1;
  const int n0 = gs * HS_NS;
  float k2[HS_NS], h[HS_NS];
#pragma unroll
  for (int s = 0; s < HS_NS; ++s) {
    k2[s] = p.A[n0 + s] * LOG2E;
    h[s] = (on && p.init_state) ? p.init_state[((int64_t)b * p.d_inner + c) * N + n0 + s] : 0.f;
  }
  const float bias = p.dt_bias ? p.dt_bias[cc] : 0.f;
  const T* xp = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + cc;
  const float* dtp = p.dt + (int64_t)b * p.dt_sb + cc;
  const T* Bp = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + n0;
  float* part = p.hs_part + ((int64_t)b * ncb + cblk) * p.seqlen * N + n0;
  // the next block's dt, x (every thread) and B (threads < HS_TB) in registers while the current one computes
  float dn[HS_TB], xn[HS_TB];
  float4 bn = {0.f, 0.f, 0.f, 0.f};
  auto load = [&](int t0) {
#pragma unroll
    for (int j = 0; j < HS_TB; ++j) {
      const int t = min(t0 + j, p.seqlen - 1);
      dn[j] = dtp[(int64_t)t * p.dt_sl];
      xn[j] = to_f32(xp[(int64_t)t * p.x_sl]);
    }
    if (tid < HS_TB) {
      const T* bp = Bp + (int64_t)min(t0 + tid, p.seqlen - 1) * p.B_sl;
      bn = float4{to_f32(bp[0]), to_f32(bp[1]), to_f32(bp[2]), to_f32(bp[3])};
    }
  };
  const int nblk = (p.seqlen + HS_TB - 1) / HS_TB;
  if (nblk > 0) {
    load(0);
    if (tid < HS_TB) sB[0][tid] = bn;
    __syncthreads();
  }
  static_assert(HS_TB * HS_NS == 64, "one value of the block per lane after the reduce-scatter");
  for (int k = 0; k < nblk; ++k) {
    // the block's steps first (no branch per token: dt and u are 0 for a channel past d_inner or a token past
    // the sequence, whose raw values are finite clamped reads)
    float dtv[HS_TB], uu[HS_TB];
#pragma unroll
    for (int j = 0; j < HS_TB; ++j) {
      const float in = (on && k * HS_TB + j < p.seqlen) ? 1.f : 0.f;
      dtv[j] = rf_dt(p, dn[j], bias) * in;
      uu[j] = dtv[j] * xn[j];
    }
    if (k + 1 < nblk) load((k + 1) * HS_TB);
    // every token's 4 states stay one value per lane (v[4 j + s]); one reduce-scatter over the wave's 64
    // channels after the block leaves lane l the sum for token l / 4, state l % 4 (per-token sums took
    // three swaps and a DPP row sum each)
    float v[64];
#pragma unroll
    for (int j = 0; j < HS_TB; ++j) {
      const float4 b4 = sB[k & 1][j];
      const float bv[HS_NS] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int s = 0; s < HS_NS; ++s) {
        h[s] = fmaf(__builtin_amdgcn_exp2f(dtv[j] * k2[s]), h[s], uu[j] * bv[s]);
        v[HS_NS * j + s] = h[s];
      }
    }
    red[w][lane / HS_NS][lane % HS_NS] = rf_reduce_scatter64(v, lane);
    if (k + 1 < nblk && tid < HS_TB) sB[(k + 1) & 1][tid] = bn;
    __syncthreads();
    if (tid < HS_TB * HS_NS) {
      const int j = tid / HS_NS, s = tid % HS_NS;
      const int t = k * HS_TB + j;
      if (t < p.seqlen) part[(int64_t)t * N + s] = red[0][j][s] + red[1][j][s] + red[2][j][s] + red[3][j][s];
    }
    __syncthreads();
  }
}

// hs[b, t, n] = (sum over channel blocks of part) / d_inner, blocks added in order.
template <typename T>
__global__ __launch_bounds__(256) void rf_hs_reduce_kernel(RfParams p) {
  const int ncb = (p.d_inner + HS_CPB - 1) / HS_CPB;
  const int64_t per = (int64_t)p.seqlen * p.dstate;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.batch * per) return;
  const int64_t b = i / per, r = i % per;
  float s = 0.f;
  for (int k = 0; k < ncb; ++k) s += p.hs_part[(b * ncb + k) * per + r];
  reinterpret_cast<T*>(p.hs)[i] = from_f32<T>(s / (float)p.d_inner);
}

template <typename T, int N>
hipError_t launch_rf_t(const RfParams& p, hipStream_t st) {
  const int nblk = p.batch * (p.d_inner / rf_cpb<N>());
  if (nblk > 0 && (p.seqlen > 0 || p.final_state)) {
    // (an empty sequence only writes the final state: the initial state, or zero)
    if (p.z && p.seqlen > 0) hipLaunchKernelGGL((rf_scan_kernel<T, N, true>), dim3(nblk), dim3(RF_NT), 0, st, p);
    else hipLaunchKernelGGL((rf_scan_kernel<T, N, false>), dim3(nblk), dim3(RF_NT), 0, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !p.hs || p.seqlen == 0) return e;
  const int ncb = (p.d_inner + HS_CPB - 1) / HS_CPB;
  hipLaunchKernelGGL((rf_hs_kernel<T, N>), dim3(p.batch * ncb * (N / HS_NS)), dim3(RF_NT), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t tot = (int64_t)p.batch * p.seqlen * N;
  hipLaunchKernelGGL((rf_hs_reduce_kernel<T>), dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_rf_n(const RfParams& p, hipStream_t st) {
  switch (p.dstate) {
    case 16: return launch_rf_t<T, 16>(p, st);
    case 32: return launch_rf_t<T, 32>(p, st);
    case 64: return launch_rf_t<T, 64>(p, st);
    case 128: return launch_rf_t<T, 128>(p, st);
    case 256: return launch_rf_t<T, 256>(p, st);
    default: return hipErrorInvalidValue;
  }
}

// ---------------------------------------------------------------- backward
// With lam_t[c, n] the adjoint of h_t[c, n] (lam after the last token = d_final),
//     lam_t = dy_t[c] C_t[n] + dhs_t[n] / d_inner + a_{t+1} lam_{t+1},      a_t = exp(A_n dt_t[c]),
//     dx_t[c]  = dt_t[c] sum_n lam_t B_t[n] + D_c dy_t[c],
//     ddt_t[c] = (sum_n lam_t A_n a_t h_{t-1} + x_t[c] sum_n lam_t B_t[n]) * d dt / d raw,
//     dB_t[n]  = sum_c lam_t dt_t[c] x_t[c],      dC_t[n] = sum_c dy_t[c] h_t[c, n],
//     dA_n     = sum_{t, c} lam_t a_t dt_t[c] h_{t-1},   d h0 = a_0 lam_0,   dD_c = sum_t dy_t[c] x_t[c].
// Every (c, n) pair follows its own recurrences given the per-token inputs.  The sums over n (dx, ddt) and over c
// (dB, dC, dA) want opposite layouts, so two kernels walk the sequence backward in pieces of RK tokens from the
// checkpoints (the state entering each piece, written by the CKPT scan): in each piece the states and decays are
// recomputed forward into registers, then the adjoint runs backward through them.
//   rf_bwd_chan_kernel: the scan's layout (a channel's states over LPC lanes, CPB channels per workgroup); the sums
//     over n on the DPP crossbar; dx, ddt per token, and per (batch, channel) dD, d dt_bias partials and d h0.
//   rf_bwd_state_kernel: lane = channel (256 per workgroup), 4 states per lane (a workgroup per batch, channel
//     block and group of 4 states); the sums over c as in rf_hs_kernel; dB, dC per (channel block, token) and dA per
//     channel block, as partials.
//   rf_bwd_reduce_kernel / rf_bwd_param_kernel: the partials added in a fixed order (deterministic).

// d dt / d raw for dt = clamp(softplus?(raw + bias), dt_min, dt_max) (the clamp passes the gradient inside its
// closed range, as torch.clamp does).
__device__ __forceinline__ float rf_dt_chain(const RfParams& p, float raw, float bias) {
  const float u = raw + bias;
  float g = 1.f, v = u;
  if (p.dt_softplus) {
    if (u <= 20.f) g = 1.f / (1.f + __expf(-u));
    v = softplus_f(u);
  }
  if (p.has_dt_limit && !(v >= p.dt_min && v <= p.dt_max)) g = 0.f;
  return g;
}

template <int N, int RK, int CPB>
struct __align__(16) RfbChanSmem {
  // 16-byte aligned rows: a lane's consecutive states of B, C and G are 16-byte LDS reads
  __align__(16) float B[RK][N];
  __align__(16) float C[RK][N];
  __align__(16) float G[RK][N];            // G = dhs / d_inner
  float dt[RK][CPB], chain[RK][CPB], x[RK][CPB], dy[RK][CPB];
  float dx[RK][CPB], ddt[RK][CPB];
};

// Piece j's rows into LDS (0 past the end of the sequence).  Every load is unconditional at a clamped (valid)
// address and masked by a factor 0 afterwards, so that all of a thread's loads are in flight together (a select
// between a loaded value and 0 lets the compiler put each load behind its own branch and wait); a missing dy or
// dhs reads x or B instead, times 0 (finite inputs).
template <typename T, int N, int RK, int CPB>
__device__ void rfb_load_piece(const RfParams& p, RfbChanSmem<N, RK, CPB>& sm, int b, int c0, int t0) {
  constexpr int NE = RK * N / RF_NT, NC = (RK * CPB + RF_NT - 1) / RF_NT;
  static_assert(RK * N % RF_NT == 0, "whole rows of B / C per pass");
  const int tid = threadIdx.x, L = p.seqlen, di = p.d_inner;
  const T* Bp = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb;
  const T* Cp = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb;
  const T* Gp = p.dhs ? reinterpret_cast<const T*>(p.dhs) + (int64_t)b * L * N : Bp;
  const int64_t gsl = p.dhs ? N : p.B_sl;
  const float gmul = p.dhs ? 1.f / (float)di : 0.f;
  T bv[NE], cv[NE], gv[NE];
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = tid + RF_NT * k, t = e / N, n = e % N, tt = min(t0 + t, L - 1);
    bv[k] = Bp[(int64_t)tt * p.B_sl + n];
    cv[k] = Cp[(int64_t)tt * p.C_sl + n];
    gv[k] = Gp[(int64_t)tt * gsl + n];
  }
  const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb;
  const T* dyb = p.dy ? reinterpret_cast<const T*>(p.dy) + (int64_t)b * L * di : xb;
  const int64_t dysl = p.dy ? di : p.x_sl;
  const float dymul = p.dy ? 1.f : 0.f;
  float raw[NC];
  T xv[NC], dv[NC];
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int e = min(tid + RF_NT * k, RK * CPB - 1), t = e / CPB, cl = e % CPB, tt = min(t0 + t, L - 1);
    raw[k] = p.dt[(int64_t)b * p.dt_sb + (int64_t)tt * p.dt_sl + c0 + cl];
    xv[k] = xb[(int64_t)tt * p.x_sl + c0 + cl];
    dv[k] = dyb[(int64_t)tt * dysl + c0 + cl];
  }
  __builtin_amdgcn_sched_barrier(0);   // every load issued before the first use
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = tid + RF_NT * k, t = e / N, n = e % N;
    const float in = t0 + t < L ? 1.f : 0.f;
    sm.B[t][n] = to_f32(bv[k]) * in;
    sm.C[t][n] = to_f32(cv[k]) * in;
    sm.G[t][n] = to_f32(gv[k]) * (in * gmul);
  }
#pragma unroll
  for (int k = 0; k < NC; ++k) {
    const int e = tid + RF_NT * k;
    if (e < RK * CPB) {
      const int t = e / CPB, cl = e % CPB;
      const float in = t0 + t < L ? 1.f : 0.f;
      const float bias = p.dt_bias ? p.dt_bias[c0 + cl] : 0.f;
      sm.dt[t][cl] = rf_dt(p, raw[k], bias) * in;
      sm.chain[t][cl] = rf_dt_chain(p, raw[k], bias) * in;
      sm.x[t][cl] = to_f32(xv[k]) * in;
      sm.dy[t][cl] = to_f32(dv[k]) * (in * dymul);
    }
  }
}

template <typename T, int N>
__global__ __launch_bounds__(RF_NT) void rf_bwd_chan_kernel(RfParams p) {
  constexpr int LPC = rf_lpc<N>(), NS = rf_ns<N>(), CPB = rf_cpb<N>(), RK = rf_rk<N>();
  __shared__ RfbChanSmem<N, RK, CPB> sm;
  const int nper = p.d_inner / CPB;
  const int b = blockIdx.x / nper, c0 = (blockIdx.x % nper) * CPB;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int cl = (64 / LPC) * w + lane / LPC, g = lane % LPC;
  const int c = c0 + cl, n0 = g * NS, L = p.seqlen, di = p.d_inner;
  const bool ylane = g == LPC - 1;   // holds the channel's sums over n after the row sums (as in the scan)
  const int nsb = (L + RK - 1) / RK;
  float k2[NS], As[NS], lamc[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    As[s] = p.A[n0 + s];
    k2[s] = As[s] * LOG2E;
    lamc[s] = p.d_final ? p.d_final[((int64_t)b * di + c) * N + n0 + s] : 0.f;
  }
  const float Dc = p.D ? (p.D_per_channel ? p.D[c] : p.D[c / p.headdim]) : 0.f;
  float dD_acc = 0.f, db_acc = 0.f;
  for (int j = nsb - 1; j >= 0; --j) {
    const int t0 = j * RK;
    __syncthreads();                   // the previous piece's LDS no longer read
    rfb_load_piece<T, N, RK, CPB>(p, sm, b, c0, t0);
    float h[NS];
    {
      const float* ck = p.ckpt + (((int64_t)b * nsb + j) * di + c) * N + n0;
#pragma unroll
      for (int s = 0; s < NS; ++s) h[s] = ck[s];
    }
    __syncthreads();
    // forward through the piece: the state before every token and every decay
    float hp[RK][NS], av[RK][NS];
#pragma unroll
    for (int t = 0; t < RK; ++t) {
      const float dtv = sm.dt[t][cl], u = dtv * sm.x[t][cl];
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float a = __builtin_amdgcn_exp2f(dtv * k2[s]);
        hp[t][s] = h[s];
        av[t][s] = a;
        h[s] = fmaf(a, h[s], u * sm.B[t][n0 + s]);
      }
    }
    // backward through it
    if constexpr (LPC == 32 && RK == 16) {
      // every token's two sums over the states (du, qq) stay one value per lane; after each group of 8 tokens one
      // reduce-scatter over the channel's 32 lanes leaves lanes 2 m, 2 m + 1 the sum for du (m < 8) or qq (m >= 8)
      // of token t + m % 8
      float vv[16];
#pragma unroll
      for (int t = RK - 1; t >= 0; --t) {
        const float dyv = sm.dy[t][cl];
        float du = 0.f, qq = 0.f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          const float lam = lamc[s] + dyv * sm.C[t][n0 + s] + sm.G[t][n0 + s];
          du = fmaf(lam, sm.B[t][n0 + s], du);
          qq = fmaf(lam * As[s], av[t][s] * hp[t][s], qq);
          lamc[s] = av[t][s] * lam;
        }
        vv[t % 8] = du;
        vv[8 + t % 8] = qq;
        if (t % 8 == 0) {
          const float r = rf_reduce_scatter32_16(vv, lane);
          // v_permlane16_swap of the value with itself: the first row's lanes hold du (first) and, from the second
          // row, qq (second) of token t + g / 2; its even lanes finish the token
          const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(r), __float_as_uint(r), false, false);
          if (g < 16 && (g & 1) == 0) {
            const int tk = t + (g >> 1);
            const float du = __uint_as_float(pr[0]), qq = __uint_as_float(pr[1]);
            const float dyk = sm.dy[tk][cl], dtv = sm.dt[tk][cl], xv = sm.x[tk][cl];
            const float ddr = (qq + xv * du) * sm.chain[tk][cl];
            sm.dx[tk][cl] = dtv * du + Dc * dyk;
            sm.ddt[tk][cl] = ddr;
            dD_acc = fmaf(dyk, xv, dD_acc);
            db_acc += ddr;
          }
        }
      }
    } else {
#pragma unroll
    for (int t = RK - 1; t >= 0; --t) {
      const float dyv = sm.dy[t][cl];
      float du = 0.f, qq = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const float lam = lamc[s] + dyv * sm.C[t][n0 + s] + sm.G[t][n0 + s];
        du = fmaf(lam, sm.B[t][n0 + s], du);
        qq = fmaf(lam * As[s], av[t][s] * hp[t][s], qq);
        lamc[s] = av[t][s] * lam;
      }
      du = row_sum16(du);
      qq = row_sum16(qq);
      if constexpr (LPC == 32) {
        du += dppf<0x142, 0xa>(du);
        qq += dppf<0x142, 0xa>(qq);
      }
      if (ylane) {
        const float dtv = sm.dt[t][cl], xv = sm.x[t][cl];
        const float ddr = (qq + xv * du) * sm.chain[t][cl];
        sm.dx[t][cl] = dtv * du + Dc * dyv;
        sm.ddt[t][cl] = ddr;
        dD_acc = fmaf(dyv, xv, dD_acc);
        db_acc += ddr;
      }
    }
    }
    __syncthreads();
    for (int e = tid; e < RK * CPB; e += RF_NT) {
      const int t = e / CPB, q = e % CPB, tt = t0 + t;
      if (tt < L) {
        const int64_t o = ((int64_t)b * L + tt) * di + c0 + q;
        reinterpret_cast<T*>(p.dx)[o] = from_f32<T>(sm.dx[t][q]);
        p.ddt[o] = sm.ddt[t][q];
      }
    }
  }
  if (p.dh0) {
    float* o = p.dh0 + ((int64_t)b * di + c) * N + n0;
#pragma unroll
    for (int s = 0; s < NS; ++s) o[s] = lamc[s];
  }
  if constexpr (LPC == 32 && RK == 16) {
    // the first row's lanes hold the channel's partial sums over their tokens
    dD_acc = row_sum16(dD_acc);
    db_acc = row_sum16(db_acc);
    if (g == 0) {
      p.dD_part[(int64_t)b * di + c] = dD_acc;
      p.dbias_part[(int64_t)b * di + c] = db_acc;
    }
  } else if (ylane) {
    p.dD_part[(int64_t)b * di + c] = dD_acc;
    p.dbias_part[(int64_t)b * di + c] = db_acc;
  }
}

// lane = channel, states n0 .. n0 + 3 of group gs; the piece's B, C and dhs of those states in LDS.
template <typename T, int N>
__global__ __launch_bounds__(RF_NT) void rf_bwd_state_kernel(RfParams p) {
  constexpr int RK = rf_rk<N>();
  __shared__ float4 sB[RK], sC[RK], sG[RK];
  __shared__ float red[4][RK][2 * HS_NS];
  const int L = p.seqlen, di = p.d_inner;
  const int ncb = (di + HS_CPB - 1) / HS_CPB, ngs = N / HS_NS;
  const int i = rf_xcd_block();
  const int gs = i % ngs, cblk = (i / ngs) % ncb, b = i / (ngs * ncb);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = cblk * HS_CPB + tid;
  const bool on = c < di;
  const int cc = on ? c : di - 1;
  const int n0 = gs * HS_NS, nsb = (L + RK - 1) / RK;
  const bool u32 = lane & 32, u16 = lane & 16;
  float k2[HS_NS], As[HS_NS], lamc[HS_NS], dA_acc[HS_NS];
#pragma unroll
  for (int s = 0; s < HS_NS; ++s) {
    As[s] = p.A[n0 + s];
    k2[s] = As[s] * LOG2E;
    lamc[s] = (on && p.d_final) ? p.d_final[((int64_t)b * di + c) * N + n0 + s] : 0.f;
    dA_acc[s] = 0.f;
  }
  const float bias = p.dt_bias ? p.dt_bias[cc] : 0.f;
  const float inv = 1.f / (float)di;
  float h[HS_NS];
  float* dBp = p.dB_part + ((int64_t)b * ncb + cblk) * L * N + n0;
  float* dCp = p.dC_part + ((int64_t)b * ncb + cblk) * L * N + n0;
  for (int j = nsb - 1; j >= 0; --j) {
    const int t0 = j * RK;
    __syncthreads();                   // the previous piece's LDS no longer read
    if (tid < RK) {
      const int tt = t0 + tid;
      float4 bv = {0.f, 0.f, 0.f, 0.f}, cv = bv, gv = bv;
      if (tt < L) {
        const T* bp = reinterpret_cast<const T*>(p.B) + (int64_t)b * p.B_sb + (int64_t)tt * p.B_sl + n0;
        const T* cp = reinterpret_cast<const T*>(p.C) + (int64_t)b * p.C_sb + (int64_t)tt * p.C_sl + n0;
        bv = float4{to_f32(bp[0]), to_f32(bp[1]), to_f32(bp[2]), to_f32(bp[3])};
        cv = float4{to_f32(cp[0]), to_f32(cp[1]), to_f32(cp[2]), to_f32(cp[3])};
        if (p.dhs) {
          const T* gp = reinterpret_cast<const T*>(p.dhs) + ((int64_t)b * L + tt) * N + n0;
          gv = float4{to_f32(gp[0]) * inv, to_f32(gp[1]) * inv, to_f32(gp[2]) * inv, to_f32(gp[3]) * inv};
        }
      }
      sB[tid] = bv;
      sC[tid] = cv;
      sG[tid] = gv;
    }
    // this lane's channel for the piece's tokens: unconditional loads at clamped addresses, masked by factors
    // (a missing dy reads x, times 0), so that they are all in flight together
    float dtv[RK], xv[RK], dyv[RK];
    {
      float raw[RK];
      T xr[RK], dr[RK];
      const T* xb = reinterpret_cast<const T*>(p.x) + (int64_t)b * p.x_sb + cc;
      const T* dyb = p.dy ? reinterpret_cast<const T*>(p.dy) + (int64_t)b * L * di + cc : xb;
      const int64_t dysl = p.dy ? di : p.x_sl;
#pragma unroll
      for (int t = 0; t < RK; ++t) {
        const int tt = min(t0 + t, L - 1);
        raw[t] = p.dt[(int64_t)b * p.dt_sb + (int64_t)tt * p.dt_sl + cc];
        xr[t] = xb[(int64_t)tt * p.x_sl];
        dr[t] = dyb[(int64_t)tt * dysl];
      }
      const float4 hv = *reinterpret_cast<const float4*>(p.ckpt + (((int64_t)b * nsb + j) * di + cc) * N + n0);
      h[0] = hv.x; h[1] = hv.y; h[2] = hv.z; h[3] = hv.w;
      __builtin_amdgcn_sched_barrier(0);   // every load issued before the first use
      const float dymul = p.dy ? 1.f : 0.f;
#pragma unroll
      for (int t = 0; t < RK; ++t) {
        const float in = (on && t0 + t < L) ? 1.f : 0.f;
        dtv[t] = rf_dt(p, raw[t], bias) * in;
        xv[t] = to_f32(xr[t]) * in;
        dyv[t] = to_f32(dr[t]) * (in * dymul);
      }
    }
    __syncthreads();
    // forward through the piece: the state after every token (hs[t]) and every decay; hs[-1] = the entry state
    float he[HS_NS], hs[RK][HS_NS], av[RK][HS_NS];
#pragma unroll
    for (int s = 0; s < HS_NS; ++s) he[s] = h[s];
#pragma unroll
    for (int t = 0; t < RK; ++t) {
      const float4 b4 = sB[t];
      const float bb[HS_NS] = {b4.x, b4.y, b4.z, b4.w};
      const float u = dtv[t] * xv[t];
#pragma unroll
      for (int s = 0; s < HS_NS; ++s) {
        const float a = __builtin_amdgcn_exp2f(dtv[t] * k2[s]);
        av[t][s] = a;
        h[s] = fmaf(a, h[s], u * bb[s]);
        hs[t][s] = h[s];
      }
    }
    // the piece's tokens backwards, in groups of 4: each token's 4-vectors of the dB and dC sums stay one value
    // per lane (v[4 ti + s] and v[16 + 4 ti + s]) and one reduce-scatter over the wave's 64 channels after the
    // group leaves lanes 2 m, 2 m + 1 the sum for (dB | dC by m / 16, token t + (m % 16) / 4, state m % 4)
    static_assert(RK % 4 == 0, "whole groups of 4 tokens");
    float v[32];
#pragma unroll
    for (int t = RK - 1; t >= 0; --t) {
      const float4 c4 = sC[t], g4 = sG[t];
      const float cv[HS_NS] = {c4.x, c4.y, c4.z, c4.w}, gv[HS_NS] = {g4.x, g4.y, g4.z, g4.w};
      const float dx_ = dtv[t] * xv[t];
      const int ti = t % 4;
#pragma unroll
      for (int s = 0; s < HS_NS; ++s) {
        const float lam = lamc[s] + dyv[t] * cv[s] + gv[s];
        const float hprev = t > 0 ? hs[t - 1][s] : he[s];
        v[HS_NS * ti + s] = lam * dx_;
        v[16 + HS_NS * ti + s] = dyv[t] * hs[t][s];
        dA_acc[s] = fmaf(lam * av[t][s], dtv[t] * hprev, dA_acc[s]);
        lamc[s] = av[t][s] * lam;
      }
      if (ti == 0) {
        const float r = rf_reduce_scatter64_32(v, lane);
        const int m = lane >> 1;
        if ((lane & 1) == 0) red[w][t + ((m & 15) >> 2)][HS_NS * (m >> 4) + (m & 3)] = r;
      }
    }
    __syncthreads();
    if (tid < RK * 2 * HS_NS) {
      const int t = tid / (2 * HS_NS), k = tid % (2 * HS_NS), tt = t0 + t;
      if (tt < L) {
        const float v = red[0][t][k] + red[1][t][k] + red[2][t][k] + red[3][t][k];
        (k < HS_NS ? dBp : dCp)[(int64_t)tt * N + (k % HS_NS)] = v;
      }
    }
  }
  // dA over the workgroup's channels: the same reduce-scatter, then the 4 waves in order
  {
    float v2[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(dA_acc[k]), __float_as_uint(dA_acc[k + 2]),
                                                       false, false);
      v2[k] = __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
    }
    const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(v2[0]), __float_as_uint(v2[1]), false, false);
    float v1 = __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
    v1 = row_sum16(v1);
    __syncthreads();
    if ((lane & 15) == 0) red[w][0][2 * (int)u32 + (int)u16] = v1;
    __syncthreads();
    if (tid < HS_NS)
      p.dA_part[((int64_t)b * ncb + cblk) * N + n0 + tid] = red[0][0][tid] + red[1][0][tid] + red[2][0][tid] +
                                                            red[3][0][tid];
  }
}

// dB, dC (b, L, N) = the channel blocks' partials added in order.
template <typename T>
__global__ __launch_bounds__(256) void rf_bwd_reduce_kernel(RfParams p) {
  const int ncb = (p.d_inner + HS_CPB - 1) / HS_CPB;
  const int64_t per = (int64_t)p.seqlen * p.dstate;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)p.batch * per) return;
  const int64_t b = i / per, r = i % per;
  float sb = 0.f, sc = 0.f;
  for (int k = 0; k < ncb; ++k) {
    sb += p.dB_part[(b * ncb + k) * per + r];
    sc += p.dC_part[(b * ncb + k) * per + r];
  }
  reinterpret_cast<T*>(p.dB)[i] = from_f32<T>(sb);
  reinterpret_cast<T*>(p.dC)[i] = from_f32<T>(sc);
}

// dA (N), dD (like D) and d dt_bias (d_inner): partials added over batch rows (and channel blocks) in order.
__global__ __launch_bounds__(256) void rf_bwd_param_kernel(RfParams p) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int di = p.d_inner, N = p.dstate, ncb = (di + HS_CPB - 1) / HS_CPB;
  if (i < N) {
    float s = 0.f;
    for (int k = 0; k < p.batch * ncb; ++k) s += p.dA_part[(int64_t)k * N + i];
    p.dA[i] = s;
  }
  if (i < di) {
    float sd = 0.f, sb = 0.f;
    for (int b = 0; b < p.batch; ++b) {
      sd += p.dD_part[(int64_t)b * di + i];
      sb += p.dbias_part[(int64_t)b * di + i];
    }
    if (p.d_dt_bias) p.d_dt_bias[i] = sb;
    if (p.dD && p.D_per_channel) p.dD[i] = sd;
  }
  if (p.dD && !p.D_per_channel && i < di / p.headdim) {     // D per head: its channels' sums
    float sd = 0.f;
    for (int b = 0; b < p.batch; ++b)
      for (int q = 0; q < p.headdim; ++q) sd += p.dD_part[(int64_t)b * di + i * p.headdim + q];
    p.dD[i] = sd;
  }
}

template <typename T, int N>
hipError_t launch_rf_bwd_t(const RfParams& p, hipStream_t st) {
  const int nblk = p.batch * (p.d_inner / rf_cpb<N>());
  if (p.seqlen > 0) {
    hipLaunchKernelGGL((rf_scan_kernel<T, N, false, true>), dim3(nblk), dim3(RF_NT), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((rf_bwd_chan_kernel<T, N>), dim3(nblk), dim3(RF_NT), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int ncb = (p.d_inner + HS_CPB - 1) / HS_CPB;
  hipLaunchKernelGGL((rf_bwd_state_kernel<T, N>), dim3(p.batch * ncb * (N / HS_NS)), dim3(RF_NT), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t tot = (int64_t)p.batch * p.seqlen * N;
  if (tot > 0) {
    hipLaunchKernelGGL((rf_bwd_reduce_kernel<T>), dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int np = p.d_inner > N ? p.d_inner : N;
  hipLaunchKernelGGL(rf_bwd_param_kernel, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, st, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_rf_bwd_n(const RfParams& p, hipStream_t st) {
  switch (p.dstate) {
    case 16: return launch_rf_bwd_t<T, 16>(p, st);
    case 32: return launch_rf_bwd_t<T, 32>(p, st);
    case 64: return launch_rf_bwd_t<T, 64>(p, st);
    case 128: return launch_rf_bwd_t<T, 128>(p, st);
    case 256: return launch_rf_bwd_t<T, 256>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool ssd_rf_supported(int dstate) {
  return dstate == 16 || dstate == 32 || dstate == 64 || dstate == 128 || dstate == 256;
}

size_t ssd_rf_workspace_bytes(int batch, int seqlen, int d_inner, int dstate, bool h_states) {
  if (!h_states) return 0;
  const size_t ncb = (size_t)(d_inner + HS_CPB - 1) / HS_CPB;
  return align256((size_t)batch * ncb * seqlen * dstate * 4);
}

hipError_t launch_ssd_rf(const RfParams& p, hipStream_t st) {
  if (p.dtype == DT_BF16) return launch_rf_n<bf16>(p, st);
  return launch_rf_n<float>(p, st);
}

// Backward workspace: the checkpoints (b, pieces, d_inner, N), the dB and dC partials (b, channel blocks, L, N),
// the dA partials (b, channel blocks, N), and the dD / d dt_bias partials (b, d_inner), all fp32.
static size_t rf_rk_of(int dstate) { return dstate == 256 ? 8 : 16; }

size_t ssd_rf_bwd_workspace_bytes(int batch, int seqlen, int d_inner, int dstate) {
  const size_t rk = rf_rk_of(dstate), nsb = (seqlen + rk - 1) / rk;
  const size_t ncb = (size_t)(d_inner + HS_CPB - 1) / HS_CPB;
  return align256((size_t)batch * nsb * d_inner * dstate * 4) + 2 * align256((size_t)batch * ncb * seqlen * dstate * 4) +
         align256((size_t)batch * ncb * dstate * 4) + 2 * align256((size_t)batch * d_inner * 4);
}

void ssd_rf_bwd_layout(RfParams& p, void* workspace) {
  const size_t rk = rf_rk_of(p.dstate), nsb = (p.seqlen + rk - 1) / rk;
  const size_t ncb = (size_t)(p.d_inner + HS_CPB - 1) / HS_CPB;
  char* w = reinterpret_cast<char*>(workspace);
  p.ckpt = reinterpret_cast<float*>(w);
  w += align256((size_t)p.batch * nsb * p.d_inner * p.dstate * 4);
  p.dB_part = reinterpret_cast<float*>(w);
  w += align256((size_t)p.batch * ncb * p.seqlen * p.dstate * 4);
  p.dC_part = reinterpret_cast<float*>(w);
  w += align256((size_t)p.batch * ncb * p.seqlen * p.dstate * 4);
  p.dA_part = reinterpret_cast<float*>(w);
  w += align256((size_t)p.batch * ncb * p.dstate * 4);
  p.dD_part = reinterpret_cast<float*>(w);
  w += align256((size_t)p.batch * p.d_inner * 4);
  p.dbias_part = reinterpret_cast<float*>(w);
}

hipError_t launch_ssd_rf_bwd(const RfParams& p, hipStream_t st) {
  if (p.dtype == DT_BF16) return launch_rf_bwd_n<bf16>(p, st);
  return launch_rf_bwd_n<float>(p, st);
}

}  // namespace mh
