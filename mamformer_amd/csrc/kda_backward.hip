// Backward of the reference-mode KDA scan (the normalised phi-kernel linear
// attention of kda_ref_kernel) for gfx950.
//
// The reference trains LinearDiffAttention through autograd of its eager
// chunked scan (mamformer/layers/kda_diff.py:357-478).  Per head, with
// phi = elu + 1 on the first kernel_dim channels and, per 64-token chunk,
// the entering state S (dk x dv) and normaliser z (dk):
//     A[t][s]   = phi(q_t) . phi(k_s)                   (s <= t, in-chunk)
//     num_t     = sum_s A[t][s] v_s + phi(q_t) S,   n_t = sum_s A[t][s] + phi(q_t) . z + 1e-8
//     o_t       = num_t / n_t
// and with do_t the output gradient:
//     dnum_t = do_t / n_t,   dn_t = -(do_t . o_t) / n_t
//     G[t][s] = dnum_t . v_s + dn_t                      (s <= t)
//     dphi(q_t) = sum_s G[t][s] phi(k_s) + S dnum_t + dn_t z
//     dv_s      = sum_i sum_{t>=s} A_i[t][s] dnum_i,t + phi(k_s) dS
//     dphi(k_s) = sum_i sum_{t>=s} G_i[t][s] phi(q_i,t) + dS v_s + dz
//     dS <- dS + sum_i phi(q_i)^T dnum_i,  dz <- dz + sum_i phi(q_i)^T dn_i      (walking backwards)
// with dS, dz the adjoint of the state after the chunk (zero, or the final-state gradient, at the end).
// dq = dphi(q) * phi'(q) and phi'(x) = min(phi(x), 1) (e^x below 0, 1 above).
//
// kda_ref_bwd_q_kernel   grid (B*H, nq): one query stream per workgroup, forward walk: dq, and n, dn per
//                        token into the workspace (plus sum(dout . o_i) for the lambda gradient).
// kda_ref_bwd_segsum_kernel grid (nseg - 1, B*H): per sequence segment, its sum of adjoint-state
//                        contributions, so that the segments' reverse walks run side by side.
// kda_ref_bwd_kv_kernel  grid (nseg, B*H): reverse walk of one segment over the query streams (one combined
//                        stream for the differential output): dk, dv, and (segment 0) dS0, dz0.
// kda_ref_bwd_lam_kernel grid (1): d lambda per head from the per-(b, h) partial sums, fixed order.
// 8 waves per workgroup; every product is a 32x32x16 bf16 MFMA over LDS tiles whose operands are read
// along rows (two 8-byte reads) or down columns (eight 2-byte reads), so no transposed copies are kept.
#include "common.h"
#include "launch.h"
#include "tiles.h"

namespace mh {

namespace {

constexpr int BC = 64;       // tokens per chunk
constexpr int BD = 128;      // dk = dv
constexpr int P128 = 152;    // bf16 row pitch of 128-wide tiles (76 words: transposing and row reads spread over the banks)
constexpr int P64 = 72;      // bf16 row pitch of 64-wide tiles
constexpr int NT = 512;      // threads per workgroup
constexpr int SEG_PARTS = 2; // workgroups per segment in the segment-sum pass

__device__ __forceinline__ float phi_f(float x) { return x > 0.f ? x + 1.f : __expf(x); }

// Fragment whose lane row (A operand) or lane column (B operand) is row r0 + l32 of M and whose k-values
// are M[r0 + l32][k0 + KSET(half, j)].
__device__ __forceinline__ Frag<bf16> frag_row(const bf16* M, int pitch, int r0, int k0) {
  const int l = lane_id(), half = l >> 5, l32 = l & 31;
  const bf16* p = M + (r0 + l32) * pitch + k0 + 4 * half;
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 8);
  Frag<bf16> f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f.v[j] = a[j];
    f.v[4 + j] = b[j];
  }
  return f;
}
// Fragment with k-values M[k0 + KSET(half, j)][c0 + l32] (k runs down a column of M): two transposing reads.
__device__ __forceinline__ Frag<bf16> frag_col(const bf16* M, int pitch, int c0, int k0) {
  return col_frag_tr(M, pitch, c0, k0);
}

__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Inclusive prefix sum within each 16-lane row (row_shr 1, 2, 4, 8; lanes without a source add 0): lane 15 of a
// row holds the row's total.
__device__ __forceinline__ float row_sum16(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x112, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x114, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x118, 0xf, 0xf, false));
  return v;
}

// Kernel A works on centered features phi' = phi - m (m[k] = 1 for k < kernel_dim): for inputs of small
// magnitude phi is close to 1 and the gradient of q lives in the deviations, which bf16 holds to 2^-9 of
// phi' but only to 2^-9 of 1 in phi.  The state splits the same way, S = m Vsum^T + S', z = m cnt + z'
// (S' = sum phi'(k) v^T, Vsum = sum v, cnt = tokens so far), and the rank-one parts enter in fp32, where the
// large terms cancel analytically:
//     u_t = phi(q_t) S'_t  (in-chunk: sum_s Ac[t][s] v_s, Ac[t][s] = K1_s + phi'(q_t).phi'(k_s), K1_s = sum phi'(k_s))
//     a_t = phi(q_t) . z'_t,  Q_t = phi(q_t) . m,  num_t = Q_t Vsum_t + u_t,  n_t = Q_t cnt_t + a_t + 1e-8
//     R_t = dnum_t . Vsum_t + dn_t cnt_t = do_t . ((a_t + 1e-8) Vsum_t - cnt_t u_t) / n_t^2
//     dphi(q_t) = m R_t + sum_s G[t][s] phi'(k_s) + S'_prev dnum_t + dn_t z'_prev
struct QSmem {
  bf16 PQ[BC * P128];     // phi'(q)
  bf16 PK[BC * P128];     // phi'(k)
  bf16 VV[BC * P128];     // v
  bf16 DN[BC * P128];     // raw output gradient, then dnum
  bf16 AM[BC * P64];      // A'[t][s] = phi'(q_t) . phi'(k_s) (s <= t)
  bf16 GM[BC * P64];      // G[t][s] (s <= t)
  bf16 SB[BD * P128];     // S' before this chunk (bf16), transposed: row d, column k
  alignas(16) float z[2][BD];    // z' before this chunk / after it
  alignas(16) float vs[2][BD];   // Vsum
  alignas(16) float cs[2][BD];   // column sums of S' over k < kernel_dim (= sum_s K1_s v_s)
  alignas(16) float part[3][8][BD];   // per 8-token group: sums of phi'(k), v, K1 v over the chunk
  float qs[BC];           // Q_t
  alignas(16) float k1[BC];      // K1_s
  float kpre[BC];         // sum_{s <= t} K1_s (in-chunk)
  float zq[BC];           // phi(q_t) . z'
  float nr[2][BC];        // row sums of the A' tiles of s-block 0 / 1
  float dnp[4][BC];       // per d-block partial sums of do . o
  float rp[4][BC];        // per d-block partial sums of do . ((a + eps) Vsum - cnt u)
  float bp[4][BC];        // per d-block partial sums of do . Vsum
  float dnn[BC];          // dn_t
  float rr[BC];           // R_t
  float red[2][8];
};

// Kernel B walks one generalised stream per query (pair / single outputs) or one combined stream (the
// fused differential output, whose two queries share the upstream gradient dout): with per token
//     Psi_t = sum_i coef_i phi(q_i,t) / n_i,t,   Xi_t = sum_i dn_i,t phi(q_i,t),   g_t = do_t (or dout)
// (coef_i = 1, or c and -lam c), the gradients of k, v and the state are
//     dv_s      = sum_{t>=s} (phi(k_s) . Psi_t) g_t + phi(k_s) dS
//     dphi(k_s) = sum_{t>=s} (g_t . v_s) Psi_t + sum_{t>=s} Xi_t + dS v_s + dz
//     dS <- dS + Psi^T g,   dz <- dz + sum_t Xi_t
// Psi and Xi are formed in fp32 before any rounding, so the cancellation between the two queries of the
// differential output (a factor up to 1 / (1 - lam) = 100) happens in fp32.
struct KVSmem {
  bf16 PK[BC * P128];     // phi(k)
  bf16 VV[BC * P128];
  bf16 PS[BC * P128];     // Psi
  bf16 XI[BC * P128];     // Xi
  bf16 DN[BC * P128];     // g
  bf16 WT[BC * P64];      // W^T[s][t] = phi(k_s) . Psi_t   (s <= t)
  bf16 MT[BC * P64];      // M^T[s][t] = g_t . v_s          (s <= t)
  bf16 SB[BD * P128];     // dS (bf16), transposed: row d, column k
  alignas(16) float dz[BD];
  alignas(16) float part[8][BD];   // per 8-token group: sums of Xi
};

__device__ __forceinline__ void query_coef(const KdaBwdParams& q, int h, int qi, float& coef) {
  coef = 1.f;
  if (q.diff) {
    const float lam = q.f.lam_h ? q.f.lam_h[h] : q.f.lam;
    const float c = 1.f / (1.f - lam + 1e-8f);
    coef = qi == 0 ? c : -lam * c;
  }
}

// phi(x) - 1 = elu(x): x above 0, e^x - 1 at or below.  Formed as a difference its error is absolute
// (~1e-7), which is what matters here: phi' enters only through sums and products next to O(1) terms.
__device__ __forceinline__ float phic_f(float x) { return x > 0.f ? x : __expf(x) - 1.f; }

}  // namespace

__global__ __launch_bounds__(NT) void kda_ref_bwd_q_kernel(KdaBwdParams q) {
  __shared__ QSmem sm;
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  const int bh = blockIdx.x, qi = blockIdx.y;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int S = p.seqlen, kd = p.kernel_dim;
  const int64_t rowbase = (int64_t)bh * S;
  const bf16* qp = reinterpret_cast<const bf16*>(qi == 0 ? p.q1 : p.q2);
  const bf16* kp = reinterpret_cast<const bf16*>(p.k);
  const bf16* vp = reinterpret_cast<const bf16*>(p.v);
  const bf16* dop = reinterpret_cast<const bf16*>(q.diff ? q.do1 : (qi == 0 ? q.do1 : q.do2));   // null: zero
  bf16* dqp = reinterpret_cast<bf16*>(qi == 0 ? q.dq1 : q.dq2);
  float* nbuf = q.nbuf + ((int64_t)qi * nbh + bh) * S;
  float* dnbuf = q.dnbuf + ((int64_t)qi * nbh + bh) * S;
  float coef;
  query_coef(q, h, qi, coef);
  const int dt = w & 3, tt = w >> 2;     // u / do tile (d-block, t-block); S' tiles (2tt + i, dt)
  const int kt = w & 3;                  // dq tile k-block

  f32x16 Sacc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    Sacc[i] = zero16();
    if (p.init_state) {
      const float* s0 = p.init_state + (int64_t)bh * BD * BD;
#pragma unroll
      for (int r = 0; r < 16; ++r) Sacc[i][r] = s0[(32 * (2 * tt + i) + acc_row(half, r)) * BD + 32 * dt + l32];
    }
  }
  if (tid < BD) {
    // an initial state enters S' and z' (Vsum = cnt = 0)
    sm.z[0][tid] = p.init_z ? p.init_z[(int64_t)bh * BD + tid] : 0.f;
    sm.vs[0][tid] = 0.f;
    float c = 0.f;
    if (p.init_state)
      for (int k = 0; k < kd; ++k) c += p.init_state[(int64_t)bh * BD * BD + k * BD + tid];
    sm.cs[0][tid] = c;
  }
  // lambda gradient pieces: sum dout . (o - Vsum / cnt) (cancellation-free: -R~_t / (n_t cnt_t)) and, once,
  // sum dout . Vsum / cnt (the same for both queries)
  float lam_acc = 0.f, base_acc = 0.f;

  // The next chunk's q, k, v, do are loaded into registers during this chunk's state update (two 16-byte
  // chunks of each per thread: row e >> 4, columns 8 (e & 15), e = tid + 512 i), hiding their latency.
  bf16x8 tq[2], tk[2], tv[2], td[2];
  auto load_tiles = [&](int p0) {
    const int ln = min(BC, S - p0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + NT * i, t = e >> 4, c0 = (e & 15) * 8;
      const int64_t r = (rowbase + p0 + (t < ln ? t : 0)) * BD + c0;
      tq[i] = ld8(qp + r);
      tk[i] = ld8(kp + r);
      tv[i] = ld8(vp + r);
      if (dop) td[i] = ld8(dop + r);
    }
  };
  if (S > 0) load_tiles(0);

  for (int pos = 0, ci = 0; pos < S; pos += BC, ++ci) {
    const int len = min(BC, S - pos);
    const int zc = ci & 1;
    if (ci > 0 && tid < BD) {      // z', Vsum, column sums past the previous chunk (fixed-order sums)
      float a0 = sm.z[zc ^ 1][tid], a1 = sm.vs[zc ^ 1][tid], a2 = sm.cs[zc ^ 1][tid];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a0 += sm.part[0][j][tid];
        a1 += sm.part[1][j][tid];
        a2 += sm.part[2][j][tid];
      }
      sm.z[zc][tid] = a0;
      sm.vs[zc][tid] = a1;
      sm.cs[zc][tid] = a2;
    }
    // ---- phase 0: phi'(q), phi'(k), v, do tiles, Q_t and K1_s; S' into LDS
    const bool full = len == BC && kd == BD && dop != nullptr;    // no row or channel masks
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + NT * i, t = e >> 4, c0 = (e & 15) * 8;
      const bool in = t < len;
      const bf16x8 qv = tq[i], kv = tk[i], vv = tv[i];
      const bf16x8 dv = td[i];
      bf16x8 qo, ko, vo, doo;
      float qsum = 0.f, ksum = 0.f;
      if (full) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float cq = phic_f((float)qv[j]), ck = phic_f((float)kv[j]);
          qo[j] = (bf16)cq;
          ko[j] = (bf16)ck;
          qsum += cq;
          ksum += ck;
        }
        qsum += 8.f;
        vo = vv;
        doo = dv;
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const bool ch = in && c0 + j < kd;
          const float cq = ch ? phic_f((float)qv[j]) : 0.f, ck = ch ? phic_f((float)kv[j]) : 0.f;
          qo[j] = (bf16)cq;
          ko[j] = (bf16)ck;
          qsum += ch ? 1.f + cq : 0.f;
          ksum += ck;
          vo[j] = in ? vv[j] : (bf16)0.f;
          doo[j] = (in && dop) ? dv[j] : (bf16)0.f;
        }
      }
      // the token's 16 chunks are one 16-lane row: prefix sums on the DPP crossbar, the total in its last lane
      qsum = row_sum16(qsum);
      ksum = row_sum16(ksum);
      if ((e & 15) == 15) {
        sm.qs[t] = qsum;
        sm.k1[t] = ksum;
      }
      *reinterpret_cast<bf16x8*>(&sm.PQ[t * P128 + c0]) = qo;
      *reinterpret_cast<bf16x8*>(&sm.PK[t * P128 + c0]) = ko;
      *reinterpret_cast<bf16x8*>(&sm.VV[t * P128 + c0]) = vo;
      *reinterpret_cast<bf16x8*>(&sm.DN[t * P128 + c0]) = doo;
    }
    // S'^T: the lane's column d holds 4 consecutive k per accumulator group, one 8-byte store each
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (bf16)Sacc[i][4 * g + j];
        *reinterpret_cast<bf16x4*>(&sm.SB[(32 * dt + l32) * P128 + 32 * (2 * tt + i) + 8 * g + 4 * half]) = v;
      }
    lds_barrier();
    if (pos + BC < S) load_tiles(pos + BC);          // the staged registers are free: the next chunk flies all chunk

    // ---- phase 1: A' tiles (t-block, s-block) = (0,0), (1,0), (1,1) by waves 0..2, computed transposed so
    // the row sums are lane-local; in-chunk prefix sums of K1 by wave 3; phi(q_t) . z' by waves 4..7.
    // The key-only part K1_s of Ac = K1_s + A' is kept apart: both queries then round it identically, and the
    // lambda gradient, a difference of the two queries' outputs, does not see its rounding.
    if (w < 3) {
      const int st = (w == 2) ? 1 : 0, tb = (w == 0) ? 0 : 1;
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < BD / 16; ++c)
        acc = mma(frag_row(sm.PK, P128, 32 * st, 16 * c), frag_row(sm.PQ, P128, 32 * tb, 16 * c), acc);
      const int t = 32 * tb + l32;
      float rs = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (32 * st + acc_row(half, r) > t) acc[r] = 0.f;
        rs += acc[r];
      }
      rs = sum_halves(rs);
      if (half == 0) sm.nr[st][t] = rs;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = (bf16)acc[4 * g + i];
        *reinterpret_cast<bf16x4*>(&sm.AM[t * P64 + 32 * st + 8 * g + 4 * half]) = o4;
      }
    } else if (w == 3) {
      sm.kpre[l] = wave_incl_scan(sm.k1[l]);
    } else {
      const int it = tid - 256, t = it >> 2, qq = it & 3;
      float acc = 0.f;
      const bf16* row = &sm.PQ[t * P128 + 32 * qq];
#pragma unroll
      for (int c = 0; c < 32; c += 8) {
        const bf16x8 q8 = *reinterpret_cast<const bf16x8*>(row + c);
        const f32x4 z0 = *reinterpret_cast<const f32x4*>(&sm.z[zc][32 * qq + c]);
        const f32x4 z1 = *reinterpret_cast<const f32x4*>(&sm.z[zc][32 * qq + c + 4]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = 32 * qq + c + j;
          acc += (k < kd ? 1.f + (float)q8[j] : 0.f) * (j < 4 ? z0[j] : z1[j - 4]);
        }
      }
      acc = sum_quad(acc);
      if (qq == 0) sm.zq[t] = acc;
    }
    lds_barrier();

    // ---- phase 2: u^T and Vsum^T tiles (d-block dt, t-block tt), o, and per-block sums over d
    const int ns = tt == 0 ? 2 : 4;      // 16-token k-steps of the causal in-chunk products
    const int t = 32 * tt + l32;
    const bool tin = t < len;
    f32x16 u = zero16(), vsum = zero16();
#pragma unroll
    for (int c = 0; c < BD / 16; ++c)
      u = mma(frag_row(sm.SB, P128, 32 * dt, 16 * c), frag_row(sm.PQ, P128, 32 * tt, 16 * c), u);
    for (int c = 0; c < ns; ++c) {
      const Frag<bf16> vf = frag_col(sm.VV, P128, 32 * dt, 16 * c);
      u = mma(vf, frag_row(sm.AM, P64, 32 * tt, 16 * c), u);
      Frag<bf16> ones, k1f;
      float k1v[8];
      kset_vals(sm.k1, c, half, k1v);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int s_ = 16 * c + kset(half, j);
        ones.v[j] = (bf16)(s_ <= t ? 1.f : 0.f);
        k1f.v[j] = (bf16)(s_ <= t ? k1v[j] : 0.f);
      }
      vsum = mma(vf, ones, vsum);
      u = mma(vf, k1f, u);
    }
    const float Q = sm.qs[t];
    const float cnt = (float)(pos + t + 1);
    const float a = sm.nr[0][t] + (tt ? sm.nr[1][t] : 0.f) + sm.kpre[t] + sm.zq[t];
    const float n = Q * cnt + a + 1e-8f;
    const float inv = tin ? 1.f / n : 0.f;
    float raw[16];
    float part = 0.f, rpart = 0.f, bpart = 0.f;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const bf16x4 r4 = *reinterpret_cast<const bf16x4*>(&sm.DN[t * P128 + 32 * dt + 8 * g + 4 * half]);
      const f32x4 cs4 = *reinterpret_cast<const f32x4*>(&sm.cs[zc][32 * dt + 8 * g + 4 * half]);
      const f32x4 vs4 = *reinterpret_cast<const f32x4*>(&sm.vs[zc][32 * dt + 8 * g + 4 * half]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = 4 * g + i;
        const float uu = u[rr] + cs4[i];
        const float vt = vsum[rr] + vs4[i];
        raw[rr] = (float)r4[i];
        part += raw[rr] * ((Q * vt + uu) * inv);
        rpart += raw[rr] * ((a + 1e-8f) * vt - cnt * uu);
        bpart += raw[rr] * vt;
      }
    }
    part = sum_halves(part);
    rpart = sum_halves(rpart);
    bpart = sum_halves(bpart);
    if (half == 0) {
      sm.dnp[dt][t] = part;
      sm.rp[dt][t] = rpart;
      sm.bp[dt][t] = bpart;
    }
    lds_barrier();

    // ---- phase 3: dnum (in place of do), dn and R
    {
      const float dsum = sm.dnp[0][t] + sm.dnp[1][t] + sm.dnp[2][t] + sm.dnp[3][t];
      const float dn = -coef * dsum * inv;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) o4[i] = (bf16)(coef * raw[4 * g + i] * inv);
        *reinterpret_cast<bf16x4*>(&sm.DN[t * P128 + 32 * dt + 8 * g + 4 * half]) = o4;
      }
      if (dt == 0 && half == 0) {
        const float rsum = sm.rp[0][t] + sm.rp[1][t] + sm.rp[2][t] + sm.rp[3][t];
        sm.dnn[t] = dn;
        sm.rr[t] = coef * rsum * inv * inv;
        if (tin) {
          nbuf[pos + t] = n;
          dnbuf[pos + t] = dn;
          lam_acc -= rsum * inv / cnt;
          base_acc += (sm.bp[0][t] + sm.bp[1][t] + sm.bp[2][t] + sm.bp[3][t]) / cnt;
        }
      }
    }
    lds_barrier();

    // ---- phase 4: G tiles (as G^T, waves 0..2)
    if (w < 3) {
      const int st = (w == 2) ? 1 : 0, tb = (w == 0) ? 0 : 1;
      f32x16 acc = zero16();
#pragma unroll
      for (int c = 0; c < BD / 16; ++c)
        acc = mma(frag_row(sm.VV, P128, 32 * st, 16 * c), frag_row(sm.DN, P128, 32 * tb, 16 * c), acc);
      const int tg = 32 * tb + l32;
      const float dn = sm.dnn[tg];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 o4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s_ = 32 * st + 8 * g + 4 * half + i;
          o4[i] = (bf16)(s_ <= tg ? acc[4 * g + i] + dn : 0.f);
        }
        *reinterpret_cast<bf16x4*>(&sm.GM[tg * P64 + 32 * st + 8 * g + 4 * half]) = o4;
      }
    }
    lds_barrier();

    // ---- phase 5: dphi(q)^T tile (k-block kt, t-block tt) -> dq
    {
      f32x16 gq = zero16();
      for (int c = 0; c < ns; ++c)
        gq = mma(frag_col(sm.PK, P128, 32 * kt, 16 * c), frag_row(sm.GM, P64, 32 * tt, 16 * c), gq);
#pragma unroll
      for (int c = 0; c < BD / 16; ++c)
        gq = mma(frag_col(sm.SB, P128, 32 * kt, 16 * c), frag_row(sm.DN, P128, 32 * tt, 16 * c), gq);
      if (tin) {
        const float dn = sm.dnn[t], R = sm.rr[t];
        bf16* out = dqp + (rowbase + pos + t) * BD + 32 * kt;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int k0 = 8 * g + 4 * half;
          const bf16x4 ph = *reinterpret_cast<const bf16x4*>(&sm.PQ[t * P128 + 32 * kt + k0]);
          const f32x4 z4 = *reinterpret_cast<const f32x4*>(&sm.z[zc][32 * kt + k0]);
          bf16x4 o4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = 32 * kt + k0 + i;
            const float dphi = gq[4 * g + i] + z4[i] * dn + R;
            o4[i] = (bf16)(k < kd ? dphi * fminf(1.f + (float)ph[i], 1.f) : 0.f);
          }
          *reinterpret_cast<bf16x4*>(out + k0) = o4;
        }
      }
    }

    // ---- phase 6: S' += phi'(k)^T v (own tiles); z', Vsum and the column sums of S' move past the chunk
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int c = 0; c < BC / 16; ++c)
        Sacc[i] = mma(frag_col(sm.PK, P128, 32 * (2 * tt + i), 16 * c), frag_col(sm.VV, P128, 32 * dt, 16 * c),
                      Sacc[i]);
    {
      // columns 2 cp, 2 cp + 1 and tokens 8 tg .. 8 tg + 7 per thread: 4-byte row reads, K1 as two 16-byte reads
      const int cp = tid & 63, tg = tid >> 6;
      float zs[2] = {0.f, 0.f}, vsn[2] = {0.f, 0.f}, csn[2] = {0.f, 0.f};
      const f32x4 k1a = *reinterpret_cast<const f32x4*>(&sm.k1[8 * tg]);
      const f32x4 k1b = *reinterpret_cast<const f32x4*>(&sm.k1[8 * tg + 4]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int s_ = 8 * tg + u;
        const bf16x2 pk = *reinterpret_cast<const bf16x2*>(&sm.PK[s_ * P128 + 2 * cp]);
        const bf16x2 vv = *reinterpret_cast<const bf16x2*>(&sm.VV[s_ * P128 + 2 * cp]);
        const float k1s = u < 4 ? k1a[u] : k1b[u - 4];
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          const float v = (float)vv[c];
          zs[c] += (float)pk[c];
          vsn[c] += v;
          csn[c] += k1s * v;
        }
      }
      *reinterpret_cast<f32x2*>(&sm.part[0][tg][2 * cp]) = f32x2{zs[0], zs[1]};
      *reinterpret_cast<f32x2*>(&sm.part[1][tg][2 * cp]) = f32x2{vsn[0], vsn[1]};
      *reinterpret_cast<f32x2*>(&sm.part[2][tg][2 * cp]) = f32x2{csn[0], csn[1]};
    }
    lds_barrier();
  }

  if (q.diff && q.lam_part) {
    const float ws = wave_sum(lam_acc), wb = wave_sum(base_acc);
    if (l == 0) {
      sm.red[0][w] = ws;
      sm.red[1][w] = wb;
    }
    lds_barrier();
    if (tid == 0) {
      float s_ = 0.f, b_ = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        s_ += sm.red[0][i];
        b_ += sm.red[1][i];
      }
      q.lam_part[(int64_t)qi * nbh + bh] = s_;
      if (qi == 0) q.lam_part[(int64_t)q.nq * nbh + bh] = b_;
    }
  }
}

// Raw rows of one (chunk, stream) for this thread's two 16-byte chunks e = tid + NT u (row e >> 4, columns
// 8 (e & 15)): the queries folded into the stream, n and dn of the row, and the stream's output gradient.  Loaded a
// (chunk, stream) ahead, so that the global latency hides behind the current one's products.
struct StreamRaw {
  bf16x8 q[2][2];         // [u][query of the stream]
  bf16x8 g[2];
  float nb[2][2], db[2][2];
};
__device__ __forceinline__ void load_stream(const KdaBwdParams& q, StreamRaw& s, int js, int bh, int pos, int len) {
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads, S = p.seqlen;
  const int64_t rowbase = (int64_t)bh * S;
  const int nqs = q.diff ? 2 : 1;          // queries folded into this stream
  const bf16* gp = reinterpret_cast<const bf16*>(q.diff ? q.do1 : (js == 0 ? q.do1 : q.do2));
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = threadIdx.x + NT * u, t = e >> 4, c0 = (e & 15) * 8;
    const bool in = t < len;
    const int64_t r = (rowbase + pos + (in ? t : 0)) * BD + c0;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i < nqs) {
        const int qi = q.diff ? i : js;
        s.q[u][i] = ld8(reinterpret_cast<const bf16*>(qi == 0 ? p.q1 : p.q2) + r);
        const int64_t nrow = ((int64_t)qi * nbh + bh) * S + pos + t;
        s.nb[u][i] = in ? q.nbuf[nrow] : 1.f;
        s.db[u][i] = in ? q.dnbuf[nrow] : 0.f;
      }
    }
    if (gp) s.g[u] = ld8(gp + r);
  }
}
// Psi, Xi and g of stream js for the chunk (len tokens) from its raw rows into LDS (zero rows beyond len).
__device__ __forceinline__ void put_stream(const KdaBwdParams& q, KVSmem& sm, const StreamRaw& s, int js, int len,
                                           const float (&coef)[2]) {
  const int kd = q.f.kernel_dim;
  const int nqs = q.diff ? 2 : 1;
  const bool has_g = q.diff ? q.do1 != nullptr : (js == 0 ? q.do1 : q.do2) != nullptr;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = threadIdx.x + NT * u, t = e >> 4, c0 = (e & 15) * 8;
    const bool in = t < len;
    float ps[8], xi[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) ps[j] = xi[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (i < nqs) {
        const int qi = q.diff ? i : js;
        const float cf = q.diff ? coef[qi] : 1.f;
        const float sc = in ? cf / s.nb[u][i] : 0.f;
        const float dn = in ? s.db[u][i] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float ph = (c0 + j < kd) ? phi_f((float)s.q[u][i][j]) : 0.f;
          ps[j] += sc * ph;
          xi[j] += dn * ph;
        }
      }
    }
    bf16x8 po, xo, go;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      po[j] = (bf16)ps[j];
      xo[j] = (bf16)xi[j];
      go[j] = (in && has_g) ? s.g[u][j] : (bf16)0.f;
    }
    *reinterpret_cast<bf16x8*>(&sm.PS[t * P128 + c0]) = po;
    *reinterpret_cast<bf16x8*>(&sm.XI[t * P128 + c0]) = xo;
    *reinterpret_cast<bf16x8*>(&sm.DN[t * P128 + c0]) = go;
  }
}


// Sum of the contributions of one part of a segment to the adjoint state, sum_t Psi_t^T g_t and
// sum_t Xi_t over its chunks and streams, for the kv-walk of the segments before it.
// grid ((nseg - 1) * SEG_PARTS, B*H): part blockIdx.x % SEG_PARTS of segment blockIdx.x / SEG_PARTS + 1
// (segment 0's sum is never needed).
__global__ __launch_bounds__(NT) void kda_ref_bwd_segsum_kernel(KdaBwdParams q) {
  __shared__ KVSmem sm;
  const KdaParams& p = q.f;
  const int bh = blockIdx.y, seg = blockIdx.x / SEG_PARTS + 1, part = blockIdx.x % SEG_PARTS;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int nch = (p.seqlen + BC - 1) / BC;
  const int pc = (q.seg_chunks + SEG_PARTS - 1) / SEG_PARTS;
  const int c_begin = seg * q.seg_chunks + part * pc;
  const int c_end = min(min(nch, (seg + 1) * q.seg_chunks), c_begin + pc);
  const int nstream = q.diff ? 1 : q.nq;
  float coef[2];
  query_coef(q, h, 0, coef[0]);
  query_coef(q, h, 1, coef[1]);
  const int dt = w & 3, ktb = 2 * (w >> 2);
  f32x16 acc[2] = {zero16(), zero16()};
  const int c8 = tid & 15, tg = tid >> 4;   // this thread's sums of Xi: columns 8 c8 .., tokens 2 tg, 2 tg + 1
  float z8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) z8[j] = 0.f;
  StreamRaw sr;
  if (c_begin < c_end) load_stream(q, sr, 0, bh, c_begin * BC, min(BC, p.seqlen - c_begin * BC));
  for (int ci = c_begin; ci < c_end; ++ci) {
    const int pos = ci * BC, len = min(BC, p.seqlen - pos);
    for (int js = 0; js < nstream; ++js) {
      put_stream(q, sm, sr, js, len, coef);
      if (js + 1 < nstream) load_stream(q, sr, js + 1, bh, pos, len);            // the next (chunk, stream)
      else if (ci + 1 < c_end) load_stream(q, sr, 0, bh, pos + BC, min(BC, p.seqlen - pos - BC));
      lds_barrier();
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < BC / 16; ++c)
          acc[i] = mma(frag_col(sm.PS, P128, 32 * (ktb + i), 16 * c), frag_col(sm.DN, P128, 32 * dt, 16 * c), acc[i]);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const bf16x8 x = ld8(&sm.XI[(2 * tg + u) * P128 + 8 * c8]);
#pragma unroll
        for (int j = 0; j < 8; ++j) z8[j] += (float)x[j];
      }
      lds_barrier();
    }
  }
  // fixed-order sum over the 32 token pairs: the 4 of a wave by shuffles, then the 8 waves through LDS (PS is
  // no longer read)
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    z8[j] += __shfl_xor(z8[j], 16, 64);
    z8[j] = sum_halves(z8[j]);
  }
  float* zp = reinterpret_cast<float*>(sm.PS);
  if (l < 16) {
    *reinterpret_cast<f32x4*>(&zp[w * BD + 8 * c8]) = f32x4{z8[0], z8[1], z8[2], z8[3]};
    *reinterpret_cast<f32x4*>(&zp[w * BD + 8 * c8 + 4]) = f32x4{z8[4], z8[5], z8[6], z8[7]};
  }
  lds_barrier();
  float zacc = 0.f;
  if (tid < BD) {
#pragma unroll
    for (int i = 0; i < NT / 64; ++i) zacc += zp[i * BD + tid];
  }
  float* o = q.segsum + ((int64_t)(seg * SEG_PARTS + part) * p.batch * p.nheads + bh) * (BD * BD + BD);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[(32 * (ktb + i) + acc_row(half, r)) * BD + 32 * dt + l32] = acc[i][r];
  if (tid < BD) o[BD * BD + tid] = zacc;
}

__global__ __launch_bounds__(NT) void kda_ref_bwd_kv_kernel(KdaBwdParams q) {
  __shared__ KVSmem sm;
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  const int bh = blockIdx.y, seg = blockIdx.x;
  const int h = bh % p.nheads;
  const int w = wave_id(), l = lane_id(), half = l >> 5, l32 = l & 31;
  const int tid = threadIdx.x;
  const int S = p.seqlen, kd = p.kernel_dim;
  const int64_t rowbase = (int64_t)bh * S;
  const bf16* kp = reinterpret_cast<const bf16*>(p.k);
  const bf16* vp = reinterpret_cast<const bf16*>(p.v);
  const int nstream = q.diff ? 1 : q.nq;
  const int nseg = gridDim.x;
  float coef[2];
  query_coef(q, h, 0, coef[0]);
  query_coef(q, h, 1, coef[1]);
  const int dt = w & 3, ktb = 2 * (w >> 2);     // dS tiles (ktb + i, dt)
  const int x4 = w & 3, st = w >> 2;            // output tiles: dv^T (d-block x4, s-block st), dphi(k)^T (k-block x4)

  // the adjoint after this segment: the final-state gradient plus the later segments' sums (fixed order: the
  // final-state gradient, then parts j from the last down); each part's 32 values of a lane are loaded together
  f32x16 dS[2];
  {
    int eo[2][16];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) eo[i][r] = (32 * (ktb + i) + acc_row(half, r)) * BD + 32 * dt + l32;
#pragma unroll
    for (int i = 0; i < 2; ++i) dS[i] = zero16();
    if (q.d_final) {
      const float* df = q.d_final + (int64_t)bh * BD * BD;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) dS[i][r] = df[eo[i][r]];
    }
    for (int j = SEG_PARTS * nseg - 1; j >= SEG_PARTS * (seg + 1); --j) {
      const float* sp = q.segsum + ((int64_t)j * nbh + bh) * (BD * BD + BD);
      float v[2][16];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) v[i][r] = sp[eo[i][r]];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) dS[i][r] += v[i][r];
    }
  }
  if (tid < BD) {
    float a = q.d_final_z ? q.d_final_z[(int64_t)bh * BD + tid] : 0.f;
    for (int j = SEG_PARTS * nseg - 1; j >= SEG_PARTS * (seg + 1); --j)
      a += q.segsum[((int64_t)j * nbh + bh) * (BD * BD + BD) + BD * BD + tid];
    sm.dz[tid] = a;
  }

  const int nch = (S + BC - 1) / BC;
  const int c_begin = seg * q.seg_chunks, c_end = min(nch, c_begin + q.seg_chunks);
  StreamRaw sr;
  bf16x8 kr[2], vr[2];                          // the chunk's k and v rows, loaded a chunk ahead
  auto load_kv = [&](int p0) {
    const int ln = min(BC, S - p0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + NT * u, t = e >> 4, c0 = (e & 15) * 8;
      const int64_t r = (rowbase + p0 + (t < ln ? t : 0)) * BD + c0;
      kr[u] = ld8(kp + r);
      vr[u] = ld8(vp + r);
    }
  };
  if (c_end > c_begin) {
    load_stream(q, sr, 0, bh, (c_end - 1) * BC, min(BC, S - (c_end - 1) * BC));
    load_kv((c_end - 1) * BC);
  }
  for (int ci = c_end - 1; ci >= c_begin; --ci) {
    const int pos = ci * BC, len = min(BC, S - pos);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + NT * u, t = e >> 4, c0 = (e & 15) * 8;
      const bool in = t < len;
      const bf16x8 kv = kr[u], vv = vr[u];
      bf16x8 ko, vo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ko[j] = (bf16)((in && c0 + j < kd) ? phi_f((float)kv[j]) : 0.f);
        vo[j] = in ? vv[j] : (bf16)0.f;
      }
      *reinterpret_cast<bf16x8*>(&sm.PK[t * P128 + c0]) = ko;
      *reinterpret_cast<bf16x8*>(&sm.VV[t * P128 + c0]) = vo;
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (bf16)dS[i][4 * g + j];
        *reinterpret_cast<bf16x4*>(&sm.SB[(32 * dt + l32) * P128 + 32 * (ktb + i) + 8 * g + 4 * half]) = v;
      }
    lds_barrier();
    if (ci - 1 >= c_begin) load_kv(pos - BC);

    // contributions of the later chunks through dS, dz
    f32x16 gv = zero16(), gk = zero16();
#pragma unroll
    for (int c = 0; c < BD / 16; ++c) {
      gv = mma(frag_row(sm.SB, P128, 32 * x4, 16 * c), frag_row(sm.PK, P128, 32 * st, 16 * c), gv);
      gk = mma(frag_col(sm.SB, P128, 32 * x4, 16 * c), frag_row(sm.VV, P128, 32 * st, 16 * c), gk);
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sm.dz[32 * x4 + 8 * g + 4 * half]);
#pragma unroll
      for (int j = 0; j < 4; ++j) gk[4 * g + j] += d4[j];
    }

    for (int js = 0; js < nstream; ++js) {
      put_stream(q, sm, sr, js, len, coef);
      if (js + 1 < nstream) load_stream(q, sr, js + 1, bh, pos, len);            // the next (chunk, stream)
      else if (ci - 1 >= c_begin) load_stream(q, sr, 0, bh, pos - BC, min(BC, S - pos + BC));
      lds_barrier();

      // W^T (waves 0..2) and M^T (waves 3..5) tiles, (t-block, s-block) = (0,0), (1,0), (1,1)
      if (w < 6) {
        const int which = w / 3, tile = w - 3 * which;
        const int sb = tile == 2 ? 1 : 0, tb = tile == 0 ? 0 : 1;
        f32x16 acc = zero16();
        if (which == 0) {
#pragma unroll
          for (int c = 0; c < BD / 16; ++c)
            acc = mma(frag_row(sm.PS, P128, 32 * tb, 16 * c), frag_row(sm.PK, P128, 32 * sb, 16 * c), acc);
        } else {
#pragma unroll
          for (int c = 0; c < BD / 16; ++c)
            acc = mma(frag_row(sm.DN, P128, 32 * tb, 16 * c), frag_row(sm.VV, P128, 32 * sb, 16 * c), acc);
        }
        const int s_ = 32 * sb + l32;
        bf16* dst = which ? sm.MT : sm.WT;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 o4;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int tg = 32 * tb + 8 * g + 4 * half + i;
            o4[i] = (bf16)(s_ <= tg ? acc[4 * g + i] : 0.f);
          }
          *reinterpret_cast<bf16x4*>(&dst[s_ * P64 + 32 * tb + 8 * g + 4 * half]) = o4;
        }
      }
      lds_barrier();

      const int c_lo = st ? 2 : 0;     // t >= s: s-block 1 sees only t-block 1
      for (int c = c_lo; c < BC / 16; ++c) {
        gv = mma(frag_col(sm.DN, P128, 32 * x4, 16 * c), frag_row(sm.WT, P64, 32 * st, 16 * c), gv);
        gk = mma(frag_col(sm.PS, P128, 32 * x4, 16 * c), frag_row(sm.MT, P64, 32 * st, 16 * c), gk);
        Frag<bf16> ones;               // B[t][s] = 1 for t >= s: the suffix sums of Xi
#pragma unroll
        for (int j = 0; j < 8; ++j) ones.v[j] = (bf16)(16 * c + kset(half, j) >= 32 * st + l32 ? 1.f : 0.f);
        gk = mma(frag_col(sm.XI, P128, 32 * x4, 16 * c), ones, gk);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int c = 0; c < BC / 16; ++c)
          dS[i] = mma(frag_col(sm.PS, P128, 32 * (ktb + i), 16 * c), frag_col(sm.DN, P128, 32 * dt, 16 * c), dS[i]);
      {
        // columns 2 cp, 2 cp + 1 and tokens 8 tg .. 8 tg + 7 per thread (4-byte row reads)
        const int cp = tid & 63, tg = tid >> 6;
        float a[2] = {0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const bf16x2 x = *reinterpret_cast<const bf16x2*>(&sm.XI[(8 * tg + u) * P128 + 2 * cp]);
          a[0] += (float)x[0];
          a[1] += (float)x[1];
        }
        *reinterpret_cast<f32x2*>(&sm.part[tg][2 * cp]) = f32x2{a[0], a[1]};
      }
      lds_barrier();
      if (tid < BD) {
        float d = sm.dz[tid];
#pragma unroll
        for (int j = 0; j < 8; ++j) d += sm.part[j][tid];
        sm.dz[tid] = d;
      }
    }

    // the row and column of this lane from a lane index recomputed here: hoisted out of the chunk loop, the
    // per-lane row pointers were spilled, and each reload waited for every outstanding load
    const int lh = lane_id_here();
    const int s_ = 32 * st + (lh & 31), hh = lh >> 5;
    if (s_ < len) {
      bf16* dvrow = reinterpret_cast<bf16*>(q.dv) + (rowbase + pos + s_) * BD + 32 * x4;
      bf16* dkrow = reinterpret_cast<bf16*>(q.dk) + (rowbase + pos + s_) * BD + 32 * x4;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int k0 = 8 * g + 4 * hh;
        const bf16x4 ph = *reinterpret_cast<const bf16x4*>(&sm.PK[s_ * P128 + 32 * x4 + k0]);
        bf16x4 ov, ok;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ov[i] = (bf16)gv[4 * g + i];
          ok[i] = (bf16)(gk[4 * g + i] * fminf((float)ph[i], 1.f));
        }
        *reinterpret_cast<bf16x4*>(dvrow + k0) = ov;
        *reinterpret_cast<bf16x4*>(dkrow + k0) = ok;
      }
    }
    lds_barrier();
  }

  if (seg != 0) return;
  if (q.dS0) {
    float* o = q.dS0 + (int64_t)bh * BD * BD;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[(32 * (ktb + i) + acc_row(half, r)) * BD + 32 * dt + l32] = dS[i][r];
  }
  if (q.dz0 && tid < BD) q.dz0[(int64_t)bh * BD + tid] = sm.dz[tid];
}

// d lambda_h = sum_b c^2 (sum dout . o1 - (1 + 1e-8) sum dout . o2),  c = 1 / (1 - lambda_h + 1e-8):
// the derivative of (o1 - lam o2) / (1 - lam + 1e-8) (kda_diff.py:473-478), summed in a fixed order from
// P_i = sum dout . (o_i - Vsum / cnt) and B = sum dout . Vsum / cnt:  P1 - (1 + 1e-8) P2 - 1e-8 B.
__global__ __launch_bounds__(256) void kda_ref_bwd_lam_kernel(KdaBwdParams q) {
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  for (int h = threadIdx.x; h < p.nheads; h += 256) {
    const float lam = p.lam_h ? p.lam_h[h] : p.lam;
    const float c = 1.f / (1.f - lam + 1e-8f);
    float s = 0.f;
    if (p.seqlen > 0)
      for (int b = 0; b < p.batch; ++b) {
        const int bh = b * p.nheads + h;
        s += q.lam_part[bh] - (1.f + 1e-8f) * q.lam_part[nbh + bh] - 1e-8f * q.lam_part[2 * nbh + bh];
      }
    q.dlam[h] = c * c * s;
  }
}

// Empty sequence: the initial-state gradients equal the final-state ones (or zero).
__global__ __launch_bounds__(256) void kda_ref_bwd_empty_kernel(KdaBwdParams q, size_t ns, size_t nz) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (q.dS0 && i < ns) q.dS0[i] = q.d_final ? q.d_final[i] : 0.f;
  if (q.dz0 && i < nz) q.dz0[i] = q.d_final_z ? q.d_final_z[i] : 0.f;
}

// Segments of the kv-walk per (b, h): enough workgroups to cover the 256 CUs, at least 4 chunks each.
int kda_bwd_segments(int batch, int nheads, int seqlen) {
  const int nbh = batch * nheads, nch = (seqlen + BC - 1) / BC;
  int nseg = (256 + nbh - 1) / nbh;
  nseg = min(nseg, max(1, nch / 4));
  return max(1, min(nseg, 8));
}

size_t kda_bwd_workspace_bytes(int batch, int nheads, int seqlen, int nq) {
  const size_t nbh = (size_t)batch * nheads;
  const int nseg = kda_bwd_segments(batch, nheads, seqlen);
  return (2 * (size_t)nq * nbh * seqlen + (size_t)(nq + 1) * nbh +
          (size_t)SEG_PARTS * nseg * nbh * (BD * BD + BD)) * sizeof(float);
}

void kda_bwd_workspace_layout(KdaBwdParams& q, void* workspace) {
  const size_t nbh = (size_t)q.f.batch * q.f.nheads, n = (size_t)q.nq * nbh * q.f.seqlen;
  q.nbuf = reinterpret_cast<float*>(workspace);
  q.dnbuf = q.nbuf + n;
  q.lam_part = q.dnbuf + n;
  q.segsum = q.lam_part + (size_t)(q.nq + 1) * nbh;
  q.nseg = kda_bwd_segments(q.f.batch, q.f.nheads, q.f.seqlen);
  const int nch = (q.f.seqlen + BC - 1) / BC;
  q.seg_chunks = (nch + q.nseg - 1) / q.nseg;
  q.nseg = (nch + q.seg_chunks - 1) / q.seg_chunks;   // no empty trailing segment
}

hipError_t launch_kda_bwd(const KdaBwdParams& q, hipStream_t st) {
  const KdaParams& p = q.f;
  const int nbh = p.batch * p.nheads;
  if (p.seqlen == 0) {
    const size_t ns = (size_t)nbh * p.dk * p.dv, nz = (size_t)nbh * p.dk;
    hipLaunchKernelGGL(kda_ref_bwd_empty_kernel, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, st, q, ns, nz);
  } else if (kda_precise_path(p)) {
    hipError_t e = launch_kda_bwd_precise(q, st);
    if (e != hipSuccess) return e;
  } else {
    hipLaunchKernelGGL(kda_ref_bwd_q_kernel, dim3((unsigned)nbh, (unsigned)q.nq), dim3(NT), 0, st, q);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (q.nseg > 1) {
      hipLaunchKernelGGL(kda_ref_bwd_segsum_kernel, dim3((unsigned)((q.nseg - 1) * SEG_PARTS), (unsigned)nbh),
                         dim3(NT), 0, st, q);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kda_ref_bwd_kv_kernel, dim3((unsigned)q.nseg, (unsigned)nbh), dim3(NT), 0, st, q);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !q.dlam) return e;
  hipLaunchKernelGGL(kda_ref_bwd_lam_kernel, dim3(1), dim3(256), 0, st, q);
  return hipGetLastError();
}

}  // namespace mh
