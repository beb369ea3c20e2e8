// KDA linear-attention chunked scans for gfx950: the decay-gated operator
// (kda_gated_kernel) and the reference's normalised phi-kernel scan
// (kda_ref_kernel, further below).
//
//   S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t          (S: dk x dv, fp32)
//   o_t = (q1_t - lam q2_t) S_t                          (inclusive of token t)
// The differential form is linear in q, so q_e = q1 - lam q2 is formed once.
// With g = 0 this is the un-normalised causal linear attention whose
// normalised phi(x)=elu(x)+1 form is the reference's LinearDiffAttention scan
// (mamformer/layers/kda_diff.py:357-478, mamformer/kernels/triton_ssd.py:121-181).
//
// Per window of tokens (a 64-token tile, or a piece of one), with G the
// in-tile inclusive cumsum of g (per channel k), base / end its values just
// before / at the window's last token and m the midpoint of its range:
//     A^T[s][t] = sum_k (k_s e^{m-G_s})[k] (q_e,t e^{G_t-m})[k]   (s <= t)   MFMA, K = dk
//     o^T[v][t] = sum_s v^T[v][s] A^T[s][t]                                    MFMA
//               + sum_k (S[k][v] e^{m-base}) (q_e,t e^{G_t-m})[k]              MFMA (state read-out)
//     S[k][v]  <- e^{end-base} S[k][v] + sum_s (e^{end-m} k_s e^{m-G_s})[k] v_s[v]   MFMA
// Windows are cut so that the spread of G within one never exceeds KRANGE,
// which keeps every factor finite.
#include "common.h"
#include "launch.h"
#include "tiles.h"

namespace mh {

namespace {

constexpr int SEGK = 64;          // tokens per segment (max)
constexpr int DK = 128;
constexpr int DVH = 64;           // v columns per workgroup
constexpr float KRANGE = 50.f;    // max spread of G per channel within a segment

// ----------------------------------------------------------------- gated mode
// One workgroup of 8 waves per (b, h, V-half) walks the sequence in 64-token
// tiles.  The next tile's q1, q2, k, v and g are loaded into registers while
// the current tile computes, so the walk streams at memory speed.  Wave w owns v-tile vt = w & 1, t-tile tt = (w >> 1) & 1 and
// k-half kh = w >> 2: it keeps the state tiles S[kh][vt] (replicated over tt),
// computes the read-out partial of (vt, tt) over its k-half, and the kh = 1
// partials are summed through LDS.  Waves 5..7 also form the three masked
// A^T tiles while waves 0..4 transpose the token-contracted operands (k^T,
// v^T) on the MFMA unit, each transpose once per tile, shared through LDS.  A tile is one factorisation window unless the spread of G within it
// exceeds KRANGE for some channel; it is then cut into shorter windows.
constexpr int KW = 8;                 // waves per workgroup

struct KdaGatedSmem {
  float G[SEG][DK];                   // raw g of the tile (direct loads), then its in-tile inclusive cumsum
  bf16 Qt[SEG * DK];                  // q_e e^{G - m}   (Tile<bf16, DK>, zero rows outside the window)
  bf16 Kt[SEG * DK];                  // k e^{m - G}     (zero rows outside the window)
  bf16 V[SEG * DVH];                  // v[:, V-half]    (Tile<bf16, DVH>)
  Frag<bf16> A[3][2][64];             // masked A^T tiles (s0,t0), (s0,t1), (s1,t1) as B-operand fragments
  Frag<bf16> VF[2][4][64];            // v^T fragments per v-tile (lane = v, k = token 16 c + KSET)
  Frag<bf16> KF[4][4][64];            // e^{end - m}-scaled k^T fragments per k-tile (lane = channel)
  f32x16 red[2][2][64];               // read-out partials of the kh = 1 waves: vt, tt, lane
  bf16 O[4][32 * 32];                 // o blocks (vt, tt) staged for coalesced stores (XHalf rows 0..31)
  float qtot[4][DK], qmin[4][DK], qmax[4][DK];   // per token-quarter cumsum statistics
  float mm[DK], em[DK], ek[DK], eg[DK];          // window midpoint m, e^{m - base}, e^{end - m}, e^{end - base}
  int wend, cut;
};

// Register-staged q1, q2, k (two 16-byte chunks each per thread), v (one) and g (four) of a tile.
struct KdaStage {
  uint4 q1[2], q2[2], k[2], v;
  f32x4 g[4];
};

}  // namespace

__global__ __launch_bounds__(64 * KW) void kda_gated_kernel(KdaParams p) {
  __shared__ KdaGatedSmem sm;
  using TQ = Tile<bf16, DK>;
  using TV = Tile<bf16, DVH>;
  using XO = XHalf<bf16>;
  const int nbh = p.batch * p.nheads;
  int bh, vh;
  const int L = blockIdx.x;
  if ((nbh & 7) == 0) {               // keep both V-halves of a (b, h) on one XCD (ids congruent mod 8)
    bh = (L & 7) | ((L >> 4) << 3);
    vh = (L >> 3) & 1;
  } else {
    bh = L >> 1;
    vh = L & 1;
  }
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int vt = w & 1, tt = (w >> 1) & 1, kh = w >> 2;
  const int tid = threadIdx.x;
  const int S = p.seqlen;
  const float lam = p.lam_h ? p.lam_h[h] : p.lam;
  const int64_t rowbase = (int64_t)bh * S;          // token row index base in (B,H,S,*) tensors
  const bf16* q1g = reinterpret_cast<const bf16*>(p.q1);
  const bf16* q2g = reinterpret_cast<const bf16*>(p.q2);
  const bf16* kg = reinterpret_cast<const bf16*>(p.k);
  const bf16* vg = reinterpret_cast<const bf16*>(p.v);
  bf16* og = reinterpret_cast<bf16*>(p.o);
  const int v0 = vh * DVH;
  const bool has_q2 = p.q2 != nullptr, has_g = p.g != nullptr;
  Frag<bf16> id[2];
  id[0] = ident_frag<bf16>(0, half, l32);
  id[1] = ident_frag<bf16>(1, half, l32);

  // state tiles S[k][v] for k-tile 2 kh + i, v-tile vt of this V-half
  f32x16 St[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    St[i] = zero16();
    if (p.init_state) {
      const float* s0 = p.init_state + (int64_t)bh * DK * 128;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * (2 * kh + i) + acc_row(half, r);
        St[i][r] = s0[kr * 128 + v0 + 32 * vt + l32];
      }
    }
  }

  // tile loads into registers (plain loads: a direct-to-LDS load in flight would make every later LDS
  // access of the tile wait for it): q1 / q2 / k chunks e = tid + 512 i -> row e >> 4, columns 8 (e & 15);
  // v chunk tid -> row tid >> 3, columns v0 + 8 (tid & 7); g chunks e = tid + 512 i -> row e >> 5, columns 4 (e & 31)
  KdaStage stg;
  auto load_qk = [&](int pos) {
    const int last = S - 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + 512 * i;
      const int64_t off = (rowbase + min(pos + (e >> 4), last)) * DK + 8 * (e & 15);
      stg.q1[i] = *reinterpret_cast<const uint4*>(q1g + off);
      if (has_q2) stg.q2[i] = *reinterpret_cast<const uint4*>(q2g + off);
      stg.k[i] = *reinterpret_cast<const uint4*>(kg + off);
    }
  };
  auto load_gv = [&](int pos) {
    const int last = S - 1;
    stg.v = *reinterpret_cast<const uint4*>(vg + (rowbase + min(pos + (tid >> 3), last)) * 128 + v0 + 8 * (tid & 7));
    if (has_g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + 512 * i;                     // row e >> 5, columns 4 (e & 31)
        stg.g[i] = *reinterpret_cast<const f32x4*>(p.g + (rowbase + min(pos + (e >> 5), last)) * DK + 4 * (e & 31));
      }
    }
  };
  load_gv(0);
  load_qk(0);

  for (int pos = 0; pos < S; pos += SEG) {
    const int len = min(SEG, S - pos);
    wait_vmem();                                         // this tile's registers
    *reinterpret_cast<uint4*>(&sm.V[TV::chunk(tid >> 3, tid & 7)]) = stg.v;
    if (has_g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int e = tid + 512 * i;
        *reinterpret_cast<f32x4*>(&sm.G[e >> 5][4 * (e & 31)]) = stg.g[i];
      }
    }
    lds_barrier();                                       // B1: g and v rows are in LDS

    // ---- in-tile cumsum of g per channel: thread (channel kc, token quarter qq)
    {
      const int kc = tid & (DK - 1), qq = tid >> 7;
      float loc[16];
      float run = 0.f, lmin = INFINITY, lmax = -INFINITY;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = 16 * qq + i;
        const float gv = (has_g && t < len) ? sm.G[t][kc] : 0.f;   // g = 0 past the end: G stays flat
        run += gv;
        loc[i] = run;
        lmin = fminf(lmin, run);
        lmax = fmaxf(lmax, run);
      }
      sm.qtot[qq][kc] = run;
      sm.qmin[qq][kc] = lmin;
      sm.qmax[qq][kc] = lmax;
      if (tid == 0) sm.cut = 0;                          // set below (after B2), read after B3
      lds_barrier();                                     // B2
      float off = 0.f, end = 0.f, gmin = INFINITY, gmax = -INFINITY;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float tq = sm.qtot[q][kc];
        gmin = fminf(gmin, end + sm.qmin[q][kc]);
        gmax = fmaxf(gmax, end + sm.qmax[q][kc]);
        if (q < qq) off += tq;
        end += tq;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.G[16 * qq + i][kc] = loc[i] + off;
      if (qq == 0) {
        // window [0, len): base G_{-1} = 0, end = G_{len-1}, m = midpoint of the G range
        const float m = 0.5f * (gmin + gmax);
        sm.mm[kc] = m;
        sm.em[kc] = __expf(m);
        sm.ek[kc] = __expf(end - m);
        sm.eg[kc] = __expf(end);
        if (gmax - gmin > KRANGE) sm.cut = 1;            // benign race: every writer stores 1
      }
    }
    lds_barrier();                                       // B3: G, window parameters, cut flag
    const bool cut = sm.cut != 0;

    // ---- factorisation windows [a, b) of this tile
    for (int a = 0; a < len;) {
      // lane-dependent LDS addresses are recomputed per window instead of hoisted (and spilled)
      int lq = l;
      asm volatile("" : "+v"(lq));
      const int halfq = lq >> 5, l32q = lq & 31;
      int b = len;
      if (cut) {
        // longest window from a whose per-channel G spread stays within KRANGE (at least one token)
        if (tid == 0) sm.wend = len;
        lds_barrier();
        if (tid < DK) {
          float mn = INFINITY, mx = -INFINITY;
          int bad = len;
          for (int t = a; t < len; ++t) {
            const float gv = sm.G[t][tid];
            mn = fminf(mn, gv);
            mx = fmaxf(mx, gv);
            if (mx - mn > KRANGE) { bad = t; break; }
          }
          atomicMin(&sm.wend, bad);
        }
        lds_barrier();
        b = max(sm.wend, a + 1);
        if (tid < DK) {
          float mn = INFINITY, mx = -INFINITY;
          for (int t = a; t < b; ++t) {
            const float gv = sm.G[t][tid];
            mn = fminf(mn, gv);
            mx = fmaxf(mx, gv);
          }
          const float base = a ? sm.G[a - 1][tid] : 0.f, end = sm.G[b - 1][tid];
          const float m = 0.5f * (mn + mx);
          sm.mm[tid] = m;
          sm.em[tid] = __expf(m - base);
          sm.ek[tid] = __expf(end - m);
          sm.eg[tid] = __expf(end - base);
        }
        lds_barrier();
      }
      const bool last_window = (b == len);

      // Qt = q_e e^{G - m}, Kt = k e^{m - G} on rows [a, b), zero elsewhere
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = tid + 512 * i;
        const int r = e >> 4, c8 = e & 15;
        bf16x8 qo, ko;
        if (r >= a && r < b) {
          const bf16x8 x1 = __builtin_bit_cast(bf16x8, stg.q1[i]);
          const bf16x8 x2 = __builtin_bit_cast(bf16x8, stg.q2[i]);
          const bf16x8 xk = __builtin_bit_cast(bf16x8, stg.k[i]);
          const f32x4 g0 = *reinterpret_cast<const f32x4*>(&sm.G[r][8 * c8]);
          const f32x4 g1 = *reinterpret_cast<const f32x4*>(&sm.G[r][8 * c8 + 4]);
          const f32x4 m0 = *reinterpret_cast<const f32x4*>(&sm.mm[8 * c8]);
          const f32x4 m1 = *reinterpret_cast<const f32x4*>(&sm.mm[8 * c8 + 4]);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float d = (j < 4 ? g0[j] : g1[j - 4]) - (j < 4 ? m0[j] : m1[j - 4]);   // G - m
            const float qe = has_q2 ? (float)x1[j] - lam * (float)x2[j] : (float)x1[j];
            qo[j] = (bf16)(qe * __expf(d));
            ko[j] = (bf16)((float)xk[j] * __expf(-d));
          }
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) qo[j] = ko[j] = (bf16)0.f;
        }
        *reinterpret_cast<bf16x8*>(&sm.Qt[TQ::chunk(r, c8)]) = qo;
        *reinterpret_cast<bf16x8*>(&sm.Kt[TQ::chunk(r, c8)]) = ko;
      }
      lds_barrier();                                     // Qt, Kt ready; G no longer read
      const bool prefetch = last_window && pos + SEG < S;
      if (prefetch) load_gv(pos + SEG);                  // the next tile streams in behind the MFMAs

      // ---- phase 1: A^T tiles (waves 5..7), the 12 operand transposes (waves 0..4), read-out partials
      if (w < 5) {
        // jobs 0..3: v^T of (v-tile j >> 1, token tile j & 1); 4..11: k^T of (k-tile (j-4) >> 1, token tile)
        for (int j = w; j < 12; j += 5) {
          if (j < 4) {
            const int vtj = j >> 1, st = j & 1;
            const f32x16 d = mfma_transpose<bf16, bf16, DVH>(sm.V, 32 * st, 32 * vtj, id, halfq, l32q);
            sm.VF[vtj][2 * st][lq] = acc_to_frag<bf16>(d, 0);
            sm.VF[vtj][2 * st + 1][lq] = acc_to_frag<bf16>(d, 1);
          } else {
            const int kt = (j - 4) >> 1, st = (j - 4) & 1;
            const float ekl = sm.ek[32 * kt + l32q];
            const f32x16 d = mfma_transpose<bf16, bf16, DK>(sm.Kt, 32 * st, 32 * kt, id, halfq, l32q);
            sm.KF[kt][2 * st][lq] = acc_to_frag_scaled<bf16>(d, 0, ekl);
            sm.KF[kt][2 * st + 1][lq] = acc_to_frag_scaled<bf16>(d, 1, ekl);
          }
        }
      } else {
        const int it = w - 5;
        const int st = (it == 2) ? 1 : 0, ttA = (it == 0) ? 0 : 1;
        f32x16 acc = zero16();
#pragma unroll
        for (int c = 0; c < DK / 16; ++c)
          acc = mma(row_frag<bf16, bf16, DK>(sm.Kt, 32 * st + l32q, 16 * c + 8 * halfq),
                    row_frag<bf16, bf16, DK>(sm.Qt, 32 * ttA + l32q, 16 * c + 8 * halfq), acc);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * st + acc_row(halfq, r) > 32 * ttA + l32q) acc[r] = 0.f;
        sm.A[it][0][lq] = acc_to_frag<bf16>(acc, 0);
        sm.A[it][1][lq] = acc_to_frag<bf16>(acc, 1);
      }
      // o^T[v][t] = sum_k (S[k][v] e^{m_k - base_k}) Qt[t][k] over this wave's k-half, t-tile tt
      f32x16 o = zero16();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kt = 2 * kh + i;
        f32x16 sv = St[i];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 e4 = *reinterpret_cast<const f32x4*>(&sm.em[32 * kt + 8 * q + 4 * halfq]);
#pragma unroll
          for (int j = 0; j < 4; ++j) sv[4 * q + j] *= e4[j];
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
          o = mma(acc_to_frag<bf16>(sv, c), kset_frag<bf16, bf16, DK>(sm.Qt, 32 * tt + l32q, 32 * kt + 16 * c, halfq), o);
      }
      lds_barrier();                                     // A^T, v^T, k^T fragments ready
      if (prefetch) load_qk(pos + SEG);

      // ---- phase 2: intra-window term (kh = 0), partial exchange, state update
      Frag<bf16> vf[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) vf[c] = sm.VF[vt][c][lq];
      if (kh == 0) {
        if (tt == 0) {
          o = mma(vf[0], sm.A[0][0][lq], o);
          o = mma(vf[1], sm.A[0][1][lq], o);
        } else {
          o = mma(vf[0], sm.A[1][0][lq], o);
          o = mma(vf[1], sm.A[1][1][lq], o);
          o = mma(vf[2], sm.A[2][0][lq], o);
          o = mma(vf[3], sm.A[2][1][lq], o);
        }
      } else {
        sm.red[vt][tt][lq] = o;
      }
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kt = 2 * kh + i;
        Frag<bf16> kf[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) kf[c] = sm.KF[kt][c][lq];
        f32x16 acc = St[i];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 e4 = *reinterpret_cast<const f32x4*>(&sm.eg[32 * kt + 8 * q + 4 * halfq]);
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[4 * q + j] *= e4[j];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) acc = mma(kf[c], vf[c], acc);
        St[i] = acc;
      }
      lds_barrier();                                     // partials in LDS; tile fragments no longer read

      // ---- output rows [a, b) of block (vt, tt): staged, then 16-byte stores
      if (kh == 0) {
        const f32x16 other = sm.red[vt][tt][lq];
        bf16* ob = sm.O[2 * vt + tt];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c0 = 8 * q + 4 * halfq;              // 4 consecutive v columns inside one 16-byte chunk
          bf16x4 yv;
#pragma unroll
          for (int j = 0; j < 4; ++j) yv[j] = (bf16)(o[4 * q + j] + other[4 * q + j]);
          *reinterpret_cast<bf16x4*>(ob + XO::chunk(l32q, c0 >> 3) + (c0 & 7)) = yv;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int e = lq + 64 * i;
          const int r = e >> 2, c = e & 3;               // row t of the block, 16-byte chunk
          const uint4 val = *reinterpret_cast<const uint4*>(ob + XO::chunk(r, c));
          const int t = 32 * tt + r;
          if (t >= a && t < b)
            *reinterpret_cast<uint4*>(og + (rowbase + pos + t) * 128 + v0 + 32 * vt + 8 * c) = val;
        }
      }
      a = b;
    }
  }

  if (p.final_state && tt == 0) {
    float* sf_out = p.final_state + (int64_t)bh * DK * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * (2 * kh + i) + acc_row(half, r);
        sf_out[kr * 128 + v0 + 32 * vt + l32] = St[i][r];
      }
  }
}

// Empty sequence: final state (and z) = initial (or zero), written by a plain kernel (no copy or memset
// node, so a captured launch behaves the same).
__global__ __launch_bounds__(256) void kda_empty_kernel(const float* __restrict__ s0, float* __restrict__ sf, size_t ns,
                                                       const float* __restrict__ z0, float* __restrict__ zf, size_t nz) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (sf && i < ns) sf[i] = s0 ? s0[i] : 0.f;
  if (zf && i < nz) zf[i] = z0 ? z0[i] : 0.f;
}

// ---------------------------------------------------------------------------
// Reference mode: the reference's normalised linear-attention scan
// (LinearDiffAttention._linear_attention_scan, kda_diff.py:357-478, and the
// Triton kernel it dispatches to, triton_ssd.py:121-181):
//     phi(x) = elu(x) + 1 on the first kernel_dim channels (0 beyond, kda_diff.py:67-89)
//     S_t = S_{t-1} + phi(k_t)^T v_t,   z_t = z_{t-1} + phi(k_t)            (inclusive of t)
//     o_i,t = phi(q_i,t) S_t / (phi(q_i,t) z_t + 1e-8)                     (i = 1, 2)
// Outputs: the pair (o1, o2); or, with o2 == NULL and two queries, the fused
// differential combination (o1 - lam o2) / (1 - lam + 1e-8) (kda_diff.py:534-538);
// or, with q2 == NULL, the single-query o1 (triton_ssd.py:184-257).
// Same segment walk and wave split as the gated kernel with g = 0; the
// normaliser is the row sum of the masked phi(q) phi(k)^T tile plus
// phi(q) . z_prev, with z (fp32) kept in LDS.
// ---------------------------------------------------------------------------
namespace {

__device__ __forceinline__ float phi1(float x) { return x > 0.f ? x + 1.f : __expf(x); }

template <int NQ>
struct KdaRefSmem {
  static constexpr int PK = DK + 24;     // bf16 row pitch (76 words: transposing and row reads spread over the banks)
  static constexpr int PV = DVH + 32;    // 48 words: the transposing reads of V spread over the banks
  bf16 Q[NQ][SEGK * PK];                 // phi(q_i)
  bf16 Kt[SEGK * PK];                    // phi(k), zero rows beyond the segment
  bf16 V[SEGK * PV];                     // v[:, V-half], zero rows beyond the segment
  alignas(16) float z[DK];               // running sum of phi(k) before this segment
  float zq[NQ][SEGK];                    // phi(q_i,t) . z
  float nrm[NQ][3][32];                  // row sums of the masked A tiles
  AccPark red[2][NQ][2];                 // k-half 1 read-out partials: vt, query, t-tile
  Frag<bf16> A[3 * NQ][2][64];           // masked A^T tiles as B-operand fragments (bf16 high part)
  Frag<bf16> Alo[3 * NQ][2][64];         // ... and the bf16 rounding remainder (A = A + Alo to ~2^-17)
  AccPark xb[NQ == 2 ? 2 : 1][2];        // fused differential output: query 2's normalised rows (vt, tt)
};

// Threads of a reference-mode workgroup: 4 waves per query stream (v-tile x k-half each).
template <int NQ>
constexpr int kda_ref_threads = 256 * NQ;

// Register-staged raw rows of one segment: per thread 16-byte chunks of k and of each query (element
// e = tid + NT i: token e >> 4, channels 8 (e & 15) ..) and of v (token e >> 3, columns 8 (e & 7) ..).
template <int NQ>
struct KdaRefStage {
  static constexpr int KC = 4 / NQ, VC = 2 / NQ;
  bf16x8 k[KC], q[NQ][KC];
  uint4 v[VC];
};

template <int NQ>
__device__ __forceinline__ void kda_ref_load(KdaRefStage<NQ>& g, const bf16* const (&qp)[2], const bf16* kk,
                                             const bf16* vv, int64_t rowbase, int pos, int len, int v0, int tid) {
  constexpr int NT = kda_ref_threads<NQ>;
#pragma unroll
  for (int i = 0; i < KdaRefStage<NQ>::KC; ++i) {
    const int e = tid + NT * i;
    const int t = e >> 4, k0 = (e & 15) * 8;
    const int64_t r = (rowbase + pos + min(t, len - 1)) * DK + k0;
    g.k[i] = *reinterpret_cast<const bf16x8*>(kk + r);
#pragma unroll
    for (int j = 0; j < NQ; ++j) g.q[j][i] = *reinterpret_cast<const bf16x8*>(qp[j] + r);
  }
#pragma unroll
  for (int i = 0; i < KdaRefStage<NQ>::VC; ++i) {
    const int e = tid + NT * i;
    const int t = e >> 3, c0 = (e & 7) * 8;
    g.v[i] = t < len ? *reinterpret_cast<const uint4*>(vv + (rowbase + pos + t) * 128 + v0 + c0)
                     : make_uint4(0, 0, 0, 0);
  }
}

}  // namespace

// 4 NQ waves: wave w has v-tile vt = w & 1, k-half kh = (w >> 1) & 1 and query stream qw = w >> 2; the two query
// streams' waves keep their own copy of the state tiles.
template <int NQ>
__global__ __launch_bounds__(256 * NQ) void kda_ref_kernel(KdaParams p) {
  __shared__ KdaRefSmem<NQ> sm;
  using SM = KdaRefSmem<NQ>;
  using TM = bf16;
  constexpr int NT = kda_ref_threads<NQ>, NW = NT / 64;
  constexpr int KC = KdaRefStage<NQ>::KC, VC = KdaRefStage<NQ>::VC;
  const int nbh = p.batch * p.nheads;
  int bh, vh;
  const int L = blockIdx.x;
  if ((nbh & 7) == 0) {               // keep both V-halves of a (b, h) on one XCD (ids congruent mod 8)
    bh = (L & 7) | ((L >> 4) << 3);
    vh = (L >> 3) & 1;
  } else {
    bh = L >> 1;
    vh = L & 1;
  }
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int vt = w & 1, kh = (w >> 1) & 1, qw = w >> 2;
  const int tid = threadIdx.x;
  const int S = p.seqlen;
  const int kd = p.kernel_dim;
  const bool fuse_diff = (NQ == 2) && (p.o2 == nullptr);
  const float lam = p.lam_h ? p.lam_h[h] : p.lam;
  const float inv_1ml = 1.f / (1.f - lam + 1e-8f);
  const int64_t rowbase = (int64_t)bh * S;
  const bf16* const qp[2] = {reinterpret_cast<const bf16*>(p.q1), reinterpret_cast<const bf16*>(p.q2)};
  const bf16* kk = reinterpret_cast<const bf16*>(p.k);
  const bf16* vv = reinterpret_cast<const bf16*>(p.v);
  bf16* op[2] = {reinterpret_cast<bf16*>(p.o), reinterpret_cast<bf16*>(p.o2)};
  const int v0 = vh * DVH;

  f32x16 St[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    St[i] = zero16();
    if (p.init_state) {
      const float* s0 = p.init_state + (int64_t)bh * DK * 128;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * (2 * kh + i) + acc_row(half, r);
        St[i][r] = s0[kr * 128 + v0 + 32 * vt + l32];
      }
    }
  }
  if (tid < DK) sm.z[tid] = p.init_z ? p.init_z[(int64_t)bh * DK + tid] : 0.f;

  static_assert(SEGK * (DK / 8) == KC * NT && SEGK * (DVH / 8) == VC * NT, "staging covers a segment");
  KdaRefStage<NQ> stg;
  if (S > 0) kda_ref_load<NQ>(stg, qp, kk, vv, rowbase, 0, min(SEGK, S), v0, tid);
  for (int pos = 0; pos < S; pos += SEGK) {
    const int len = min(SEGK, S - pos);
    // ---- phase B: phi(q_i), phi(k), v tiles from the staged rows; then stage the next segment's rows
    auto stage = [&](auto MASKc) {     // MASK: zero tokens past the segment end and channels past kernel_dim
      constexpr bool MASK = decltype(MASKc)::value;
#pragma unroll
      for (int ie = 0; ie < KC; ++ie) {
        const int e = tid + NT * ie;
        const int t = e >> 4, k0 = (e & 15) * 8;
        const bool in = t < len;
        const bf16x8 kv8 = stg.k[ie];
        bf16x8 ko;
#pragma unroll
        for (int j = 0; j < 8; ++j) {   // computed unconditionally, then selected: no branch per element
          const float f = phi1((float)kv8[j]);
          ko[j] = (bf16)((!MASK || (in && k0 + j < kd)) ? f : 0.f);
        }
        *reinterpret_cast<bf16x8*>(&sm.Kt[t * SM::PK + k0]) = ko;
#pragma unroll
        for (int i = 0; i < NQ; ++i) {
          const bf16x8 qv8 = stg.q[i][ie];
          bf16x8 qo;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float f = phi1((float)qv8[j]);
            qo[j] = (bf16)((!MASK || (in && k0 + j < kd)) ? f : 0.f);
          }
          *reinterpret_cast<bf16x8*>(&sm.Q[i][t * SM::PK + k0]) = qo;
        }
      }
    };
    if (len == SEGK && kd >= DK) stage(std::false_type{});
    else stage(std::true_type{});
#pragma unroll
    for (int ie = 0; ie < VC; ++ie) {
      const int e = tid + NT * ie;
      const int t = e >> 3, c0 = (e & 7) * 8;
      *reinterpret_cast<uint4*>(&sm.V[t * SM::PV + c0]) = stg.v[ie];
    }
    if (pos + SEGK < S) kda_ref_load<NQ>(stg, qp, kk, vv, rowbase, pos + SEGK, min(SEGK, S - pos - SEGK), v0, tid);
    __syncthreads();

    // ---- phase B2: phi(q_i,t) . z_prev  (4 adjacent lanes per (query, token), 32 channels each: one item
    // per thread)
    {
      const int it = tid;
      const int i = it / (SEGK * 4), t = (it >> 2) % SEGK, qq = it & 3;
      const bf16* row = &sm.Q[i][t * SM::PK + 32 * qq];
      float acc = 0.f;
#pragma unroll
      for (int c = 0; c < 32; c += 8) {
        const bf16x8 q8 = *reinterpret_cast<const bf16x8*>(row + c);
        const f32x4 z0 = *reinterpret_cast<const f32x4*>(&sm.z[32 * qq + c]);
        const f32x4 z1 = *reinterpret_cast<const f32x4*>(&sm.z[32 * qq + c + 4]);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += (float)q8[j] * (j < 4 ? z0[j] : z1[j - 4]);
      }
      acc = sum_quad(acc);
      if (qq == 0) sm.zq[i][t] = acc;
    }

    // ---- phase C: masked A^T tiles (query, s-tile, t-tile) and their row sums
    for (int ti = w; ti < 3 * NQ; ti += NW) {
      const int qi = ti / 3, tile = ti - 3 * qi;
      const int st = (tile == 2) ? 1 : 0, tt = (tile == 0) ? 0 : 1;
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < DK / 16; ++c) {
        Frag<TM> a, bb;
        a.v = *reinterpret_cast<const bf16x8*>(&sm.Kt[(32 * st + l32) * SM::PK + 16 * c + 8 * half]);
        bb.v = *reinterpret_cast<const bf16x8*>(&sm.Q[qi][(32 * tt + l32) * SM::PK + 16 * c + 8 * half]);
        acc = mma(a, bb, acc);
      }
      const int tl = 32 * tt + l32;
      float rs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int s_ = 32 * st + acc_row(half, r);
        if (!(s_ <= tl && s_ < len)) acc[r] = 0.f;
        rs += acc[r];
      }
      rs = sum_halves(rs);
      if (half == 0) sm.nrm[qi][tile][l32] = rs;
      // The normaliser uses the fp32 row sums, so the weights that multiply v must carry
      // more than bf16 precision or their rounding (independent per entry) does not cancel
      // against it; the differential combination can amplify that by 1/(1 - lam) <= 100.
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        Frag<TM> hi, lo;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = acc[8 * c + j];
          hi.v[j] = (bf16)x;
          lo.v[j] = (bf16)(x - (float)hi.v[j]);
        }
        sm.A[ti][c][l] = hi;
        sm.Alo[ti][c][l] = lo;
      }
    }
    __syncthreads();

    // ---- z update (z_prev was consumed by phase B2 before the barrier)
    // by the k-half 0 waves, whose read-out phase below has half the intra-segment MFMAs of the k-half 1 waves;
    // one lane per channel, in token order
    if (tid < DK) {
      float zs = 0.f;
#pragma unroll 8
      for (int t = 0; t < SEGK; ++t) zs += (float)sm.Kt[t * SM::PK + tid];
      sm.z[tid] += zs;
    }

    // ---- phase D: per wave (v-tile vt, k-half kh)
    Frag<TM> vf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) vf[c] = col_frag_tr(sm.V, SM::PV, 32 * vt, 16 * c);

    // read-out of this wave's query stream qw: o[tt] for both t-tiles over this wave's k-half
    f32x16 o[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int kt = 2 * kh + i;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const Frag<TM> sa = acc_to_frag<TM>(St[i], c);
          Frag<TM> qb;
          const bf16* row = &sm.Q[qw][(32 * tt + l32) * SM::PK + 32 * kt + 16 * c];
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(row + 4 * half);
          const bf16x4 hi = *reinterpret_cast<const bf16x4*>(row + 8 + 4 * half);
#pragma unroll
          for (int j = 0; j < 4; ++j) { qb.v[j] = lo[j]; qb.v[4 + j] = hi[j]; }
          acc = mma(sa, qb, acc);
        }
      }
      o[tt] = acc;
    }
    // wave kh finishes token tile tt = kh: it adds the intra-segment term of that tile and hands its
    // read-out partial of the other tile to the partner wave (same vt and query, other k-half)
    if (kh == 0) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        o[0] = mma(vf[c], sm.A[3 * qw + 0][c][l], o[0]);
        o[0] = mma(vf[c], sm.Alo[3 * qw + 0][c][l], o[0]);
      }
      park_acc(sm.red[vt][qw][1], o[1], l);
    } else {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        o[1] = mma(vf[c], sm.A[3 * qw + 1][c][l], o[1]);
        o[1] = mma(vf[c], sm.Alo[3 * qw + 1][c][l], o[1]);
        o[1] = mma(vf[2 + c], sm.A[3 * qw + 2][c][l], o[1]);
        o[1] = mma(vf[2 + c], sm.Alo[3 * qw + 2][c][l], o[1]);
      }
      park_acc(sm.red[vt][qw][0], o[0], l);
    }
    // state update (no decay): S[k][v] += sum_s phi(k_s)[k] v_s[v]
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int kt = 2 * kh + i;
      f32x16 acc = St[i];
#pragma unroll
      for (int c = 0; c < 4; ++c) acc = mma(col_frag_tr(sm.Kt, SM::PK, 32 * kt, 16 * c), vf[c], acc);
      St[i] = acc;
    }
    __syncthreads();
    // normalised rows of token tile tt = kh for query qw
    float res[16];
    const int tl = 32 * kh + l32;
    const bool valid = tl < len;
    auto finish = [&](auto TTc) {
      constexpr int tt = decltype(TTc)::value;
      if (valid) {
        const float nr = sm.zq[qw][tl] + (tt == 0 ? sm.nrm[qw][0][l32] : sm.nrm[qw][1][l32] + sm.nrm[qw][2][l32]);
        const float inv = 1.f / (nr + 1e-8f);
        const f32x16 other = unpark_acc(sm.red[vt][qw][tt], l);
#pragma unroll
        for (int r = 0; r < 16; ++r) res[r] = (o[tt][r] + other[r]) * inv;
      }
    };
    if (kh == 0) finish(std::integral_constant<int, 0>{});
    else finish(std::integral_constant<int, 1>{});
    if (!fuse_diff) {
      if (valid) {
        bf16* orow = op[qw] + (rowbase + pos + tl) * 128 + v0 + 32 * vt;
#pragma unroll
        for (int r = 0; r < 16; ++r) orow[acc_row(half, r)] = (bf16)res[r];
      }
      __syncthreads();
    } else {
      // the differential combination (o1 - lam o2) / (1 - lam + 1e-8): query 2's waves hand their rows over
      if (qw == 1 && valid) park_acc(sm.xb[vt][kh], res, l);
      __syncthreads();
      if (qw == 0 && valid) {
        bf16* orow = op[0] + (rowbase + pos + tl) * 128 + v0 + 32 * vt;
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
          const f32x4 r2 = sm.xb[vt][kh].p[r >> 2][l];
#pragma unroll
          for (int j = 0; j < 4; ++j) orow[acc_row(half, r + j)] = (bf16)((res[r + j] - lam * r2[j]) * inv_1ml);
        }
      }
    }
  }

  if (p.final_state && qw == 0) {
    float* sf_out = p.final_state + (int64_t)bh * DK * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kr = 32 * (2 * kh + i) + acc_row(half, r);
        sf_out[kr * 128 + v0 + 32 * vt + l32] = St[i][r];
      }
  }
  if (p.final_z && vh == 0 && tid < DK) p.final_z[(int64_t)bh * DK + tid] = sm.z[tid];
}

hipError_t launch_kda(const KdaParams& p, hipStream_t st) {
  const int nbh = p.batch * p.nheads;
  if (p.seqlen == 0) {
    const size_t ns = p.final_state ? (size_t)nbh * p.dk * p.dv : 0, nz = p.final_z ? (size_t)nbh * p.dk : 0;
    const size_t n = ns > nz ? ns : nz;
    if (n) hipLaunchKernelGGL(kda_empty_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p.init_state,
                              p.final_state, ns, p.init_z, p.final_z, nz);
    return hipGetLastError();
  }
  if (kda_precise_path(p)) return launch_kda_precise(p, st);
  const dim3 grid((unsigned)(2 * nbh));
  if (p.mode == 0) {
    hipLaunchKernelGGL(kda_gated_kernel, grid, dim3(64 * KW), 0, st, p);
  } else if (p.q2) {
    hipLaunchKernelGGL(kda_ref_kernel<2>, grid, dim3(kda_ref_threads<2>), 0, st, p);
  } else {
    hipLaunchKernelGGL(kda_ref_kernel<1>, grid, dim3(kda_ref_threads<1>), 0, st, p);
  }
  return hipGetLastError();
}

}  // namespace mh
