// Internal (not exported) kernel parameter blocks and launchers.  The C ABI in
// capi.hip validates the public argument structs, fills these and launches.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

enum { DT_F32 = 0, DT_BF16 = 1 };

// ------------------------------------------------------------- decode
struct SsuParams {
  int batch, nheads, headdim, dstate, ngroups, dtype;
  int dt_softplus, has_dt_limit, D_per_channel;
  int A_per_state, dt_per_channel;           // the reference's per-state A / per-channel dt
  float dt_min, dt_max;
  const float* state_in;
  float* state_out;
  const void* x; int64_t x_stride_b;
  const float* dt; int64_t dt_stride_b;
  const float* A;
  const void* B; int64_t B_stride_b;
  const void* C; int64_t C_stride_b;
  const float* D;
  const float* dt_bias;
  void* y; int64_t y_stride_b;
  const void* z; int64_t z_stride_b;       // optional gate: y <- y * silu(z)
};
hipError_t launch_ssu(const SsuParams& p, hipStream_t st);

// ------------------------------------------------------------- SSD prefill
struct SsdParams {
  int batch, seqlen, nheads, headdim, dstate, ngroups, dtype;
  int chunk_len;       // state-passing chunk length (multiple of 64)
  int nchunks;         // ceil(seqlen / chunk_len)
  int heads_per_wg;    // heads handled by one workgroup (one wave per head)
  int dt_softplus, has_dt_limit, D_per_channel;
  float dt_min, dt_max;
  const void* x; int64_t x_sb, x_sl, x_sh;
  const float* dt; int64_t dt_sb, dt_sl;
  const float* A;
  const void* B; int64_t B_sb, B_sl;
  const void* C; int64_t C_sb, C_sl;
  const float* D;
  const float* dt_bias;
  const float* init_state;
  void* y; int64_t y_sb, y_sl, y_sh;
  const void* z; int64_t z_sb, z_sl, z_sh; // optional gate: y <- y * silu(z)
  float* final_state;
  float* chunk_states;   // workspace: [batch][nchunks][nheads][headdim][dstate] (bf16 elements for bf16 I/O)
  float* chunk_decay;    // workspace: [batch][nheads][nchunks]  (sum of A*dt over the chunk)
  void* seg_frags;       // workspace: [batch][ngroups][nseg] shared MFMA fragments of each 64-token segment
  void* entering;        // workspace (bf16 I/O): bf16 entering states, chunk_states order
  int nseg;              // ceil(seqlen / 64)
  int state_perm;        // workspace states in state_row_perm row order (two-pass prefill)
  float* xsum;           // optional (b, L, H, 2): sums of x over each half of a head's 64 channels per token
                         // (written by the prefill, read by h_states instead of x)
};
// xsum from x by a separate pass (prefill paths whose scan does not write it).
hipError_t launch_ssd_xsum(const SsdParams& p, hipStream_t st);
hipError_t launch_ssd(const SsdParams& p, hipStream_t st);
// The two-pass bf16 prefill (ssd_lookback.hip): sizes it implements, and its launch.
bool ssd_lb_supported(int dtype, int dstate);
hipError_t launch_ssd_lb(const SsdParams& p, hipStream_t st);
// Entering states from chunk states (ssd_state_pass_kernel): H_0 = h0, H_{k+1} = e^{T_k} H_k + S_k.
hipError_t launch_ssd_state_pass(const SsdParams& p, hipStream_t st);
size_t ssd_frag_bytes(int dtype, int dstate);
size_t ssd_workspace_bytes(int batch, int seqlen, int nchunks, int nheads, int headdim, int dstate, int ngroups,
                           int dtype);
// Point p's workspace parts into `workspace` (ssd_workspace_bytes of p's sizes).
void ssd_workspace_layout(SsdParams& p, void* workspace);

// The reference's own scan form (ssd_refform.hip): a decay rate per state (A (N,), negative) and a step size per
// channel (dt (b, L, d_inner)), one group of B / C; x, y, z (b, L, d_inner) with contiguous channels.
struct RfParams {
  int batch, seqlen, d_inner, headdim, dstate, dtype;
  int dt_softplus, has_dt_limit, D_per_channel;
  float dt_min, dt_max;
  const void* x; int64_t x_sb, x_sl;
  const float* dt; int64_t dt_sb, dt_sl;
  const float* A;            // (N,) decay rates
  const void* B; int64_t B_sb, B_sl;
  const void* C; int64_t C_sb, C_sl;
  const float* D;            // (d_inner,) or (d_inner / headdim,) or null
  const float* dt_bias;      // (d_inner,) or null
  const float* init_state;   // (b, d_inner, N) or null
  void* y; int64_t y_sb, y_sl;
  const void* z; int64_t z_sb, z_sl;   // optional gate
  float* final_state;        // (b, d_inner, N) or null
  void* hs;                  // (b, L, N) h_states in the I/O dtype, or null
  float* hs_part;            // workspace: per-channel-block sums of the states, (b, blocks, L, N)
  // backward (launch_ssd_rf_bwd): upstream gradients, outputs, and the workspace pieces
  const void* dy;            // (b, L, d_inner) contiguous, I/O dtype, or null (zero)
  const void* dhs;           // (b, L, N) contiguous, I/O dtype, or null
  const float* d_final;      // (b, d_inner, N) or null
  void* dx;                  // (b, L, d_inner) contiguous, I/O dtype
  float* ddt;                // (b, L, d_inner) contiguous, w.r.t. the raw dt
  float* dA;                 // (N,) w.r.t. the rates A
  void* dB; void* dC;        // (b, L, N) contiguous, I/O dtype
  float* dD;                 // like D, or null
  float* d_dt_bias;          // (d_inner,) or null
  float* dh0;                // (b, d_inner, N) or null
  float* ckpt;               // workspace: (b, pieces, d_inner, N) the state entering every piece of the sequence
  float* dB_part; float* dC_part;   // workspace: (b, channel blocks, L, N) sums over a block's channels
  float* dA_part;            // workspace: (b, channel blocks, N)
  float* dD_part; float* dbias_part;  // workspace: (b, d_inner) sums over the tokens of one batch row
};
bool ssd_rf_supported(int dstate);
size_t ssd_rf_workspace_bytes(int batch, int seqlen, int d_inner, int dstate, bool h_states);
hipError_t launch_ssd_rf(const RfParams& p, hipStream_t st);
// Backward of the reference-form scan: checkpoints (a forward pass), the gradients, fixed-order reductions.
size_t ssd_rf_bwd_workspace_bytes(int batch, int seqlen, int d_inner, int dstate);
void ssd_rf_bwd_layout(RfParams& p, void* workspace);
hipError_t launch_ssd_rf_bwd(const RfParams& p, hipStream_t st);

// h_states of the prefill (ssd_hstates.hip): mean over (h, p) of the state after every token.
struct HsParams {
  void* hs;                  // (b, L, N) in the I/O dtype
  float* z;                  // workspace: (b, nseg, H, N) per-segment state sums (local, then entering)
  float* dec;                // workspace: (b, nseg, H) segment decays
  float* u;                  // workspace: (b, L, H) sum_p x (backward); e^{c} per (token, head) (forward)
  float* w;                  // workspace, forward: (b, nseg, G, 32, 32) the segments' in-segment weights W_g[t][s]
  // backward
  const void* dhs;           // (b, L, N) gradient of h_states, I/O dtype
  void* dx;                  // (b, L, H, P) contiguous, I/O dtype
  float* ddt;                // (b, L, H) fp32 (w.r.t. the raw dt)
  float* dA;                 // (H,)
  void* dB;                  // (b, L, G, N) contiguous, I/O dtype
  float* d_dt_bias;          // (H,) or null
  float* dx_rows;            // (b, L, H) fp32 or null: dx written once per (token, head) row instead of into dx
  float* lam;                // workspace: (b, nseg, H, N) the adjoint's local parts, then the adjoint entering
  float* part;               // workspace: (b, nseg, H, 2) dA and d_dt_bias partials
};
bool ssd_hs_supported(int nheads, int dstate);
bool ssd_hs_bwd_supported(int nheads, int dstate);
size_t ssd_hs_workspace_bytes(int batch, int seqlen, int nheads, int dstate, int ngroups, bool backward);
// Lays out q's workspace parts and sets p.nseg to this pass's segment count.
void ssd_hs_workspace_layout(SsdParams& p, HsParams& q, void* workspace, bool backward);
hipError_t launch_ssd_hs(const SsdParams& p, const HsParams& q, hipStream_t st);
// Gradients of <dhs, h_states> w.r.t. x, dt (raw), A, B, dt_bias and the initial state (dh0, (b, H, P, N), may
// be null).
hipError_t launch_ssd_hs_bwd(const SsdParams& p, const HsParams& q, float* dh0, hipStream_t st);

// ------------------------------------------------------------- SSD prefill backward
struct SsdBwdParams {
  SsdParams f;               // forward sizes and inputs (no forward workspace)
  const void* dy; int64_t dy_sb, dy_sl, dy_sh;
  const float* d_final;      // (b, H, P, N) fp32 or null
  void* dx; int64_t dx_sb, dx_sl, dx_sh;
  float* ddt; int64_t ddt_sb, ddt_sl;     // gradient w.r.t. the raw dt
  float* dA;                 // (H,)
  float* dD;                 // (H,) or (H*P,) or null
  float* dbias;              // (H,) or null
  float* dh0;                // (b, H, P, N) or null
  void* dB; int64_t dB_sb, dB_sl;
  void* dC; int64_t dC_sb, dC_sl;
  float* dB_part;            // workspace: per head block of a group, (b, L, G, N) fp32 sums over its heads
  float* dC_part;
  void* hin;                 // workspace: state entering every 64-token segment, (b, nseg, H) x fragment order
  void* lam;                 // workspace: adjoint of the state leaving every segment, same layout
  float* part_s;             // workspace: (b, nseg, H, 3) per-segment dA, d_dt_bias, dD (per head) partials
  float* part_dc;            // workspace: (b, nseg, H, 2, P) per-segment, per-token-half dD partials (per channel)
  int heads_per_wg;          // heads of one group handled by a workgroup of the gradient kernel (HB)
  const float* dx_rows;      // (b, L, H) fp32 or null: added to every channel of dx[b, t, h, :]
};
hipError_t launch_ssd_bwd(const SsdBwdParams& p, hipStream_t st);
size_t ssd_bwd_workspace_bytes(int batch, int seqlen, int nheads, int dstate, int ngroups, int dtype,
                               int heads_per_wg, int d_per_channel);
void ssd_bwd_workspace_layout(SsdBwdParams& p, void* workspace);

// ------------------------------------------------------------- KDA
struct KdaParams {
  int batch, nheads, seqlen, dk, dv, dtype;
  int mode;            // 0 gated, 1 reference (phi + normaliser)
  int kernel_dim;      // reference mode: phi applied to the first kernel_dim channels
  float lam;           // gated mode: scalar lambda
  const float* lam_h;  // per-head lambda (overrides lam when set)
  const void* q1; const void* q2; const void* k; const void* v;
  const float* g;      // gated mode: per-channel log decay (B,H,S,dk) fp32, may be null (no decay)
  const float* init_state;   // (B,H,dk,dv) fp32 or null
  const float* init_z;       // reference mode: (B,H,dk) fp32 or null
  float* final_state;        // (B,H,dk,dv) fp32 or null
  float* final_z;            // reference mode: (B,H,dk) or null
  void* o;                   // gated: o; reference: o1
  void* o2;                  // reference: o2
};
hipError_t launch_kda(const KdaParams& p, hipStream_t st);

// Backward of the reference-mode scan (kda_backward.hip).
struct KdaBwdParams {
  KdaParams f;               // forward inputs (mode 1; o, o2, final_state, final_z unused)
  int nq;                    // query streams (1 or 2)
  int diff;                  // 1: do1 is the gradient of the fused (o1 - lam o2) / (1 - lam + 1e-8)
  const void* do1; const void* do2;     // (B,H,S,dv) in the I/O dtype; null = zero
  const float* d_final;      // (B,H,dk,dv) gradient of the final state, or null
  const float* d_final_z;    // (B,H,dk) gradient of the final normaliser, or null
  void* dq1; void* dq2; void* dk; void* dv;   // (B,H,S,dk) / (B,H,S,dv) in the I/O dtype
  float* dS0;                // (B,H,dk,dv) or null
  float* dz0;                // (B,H,dk) or null
  float* dlam;               // (H,) or null (diff mode)
  float* nbuf; float* dnbuf; // workspace: n_t and dn_t per (query, b, h, token)
  float* lam_part;           // workspace: sum dout . o_i per (query, b, h)
  float* segsum;             // workspace: per (segment, b, h) adjoint-state sums (dk*dv + dk floats)
  int nseg, seg_chunks;      // kv-walk segments per (b, h) and 64-token chunks per segment
};
hipError_t launch_kda_bwd(const KdaBwdParams& q, hipStream_t st);
// fp32-arithmetic kernels (kda_precise.hip) for everything but bf16 with dk = dv = 128; launch_kda and
// launch_kda_bwd route there.
bool kda_precise_path(const KdaParams& p);
hipError_t launch_kda_precise(const KdaParams& p, hipStream_t st);
hipError_t launch_kda_bwd_precise(const KdaBwdParams& q, hipStream_t st);
size_t kda_bwd_workspace_bytes(int batch, int nheads, int seqlen, int nq);
void kda_bwd_workspace_layout(KdaBwdParams& q, void* workspace);

// ------------------------------------------------------------- KDA one-token step
struct KdaStepParams {
  int batch, nheads, dk, dv, dtype;
  int kernel_dim;            // phi applied to the first kernel_dim channels (apply_phi)
  int apply_phi;             // 1: q/k are raw, apply phi in the kernel; 0: already feature-mapped
  float lam;
  const float* lam_h;
  const void* q1; const void* q2; const void* k; const void* v;   // (B,H,dk) / (B,H,dv) contiguous
  float* state;              // (B,H,dk,dv) fp32, in place
  float* z;                  // (B,H,dk) fp32, in place
  void* o;                   // (B,H,dv): fused diff output, or o1
  void* o2;                  // optional o2 (pair)
};
hipError_t launch_kda_step(const KdaStepParams& p, hipStream_t st);

// ------------------------------------------------------------- causal conv1d
struct Conv1dParams {
  int batch, seqlen, dim, width, dtype, silu;
  int cs_len;                  // rows of conv_state (0 .. width-1)
  const void* x; int64_t x_sb, x_sl;
  const float* weight;         // (dim, width) fp32
  const float* bias;           // (dim,) fp32 or null
  const void* conv_state; int64_t cs_sb, cs_sl;
  void* y; int64_t y_sb, y_sl;
};
hipError_t launch_conv1d(const Conv1dParams& p, hipStream_t st);

struct Conv1dBwdParams {
  Conv1dParams f;              // forward inputs (y unused)
  const void* dy; int64_t dy_sb, dy_sl;
  void* dx; int64_t dx_sb, dx_sl;
  float* dweight;              // (dim, width)
  float* dbias;                // (dim,) or null
  void* dcs; int64_t dcs_sb, dcs_sl;   // gradient of the cs_len cached rows, or null
  float* dw_part;              // workspace: per (batch, 32-token run) partial sums
  float* db_part;
};
hipError_t launch_conv1d_bwd(const Conv1dBwdParams& q, hipStream_t st);
size_t conv1d_bwd_workspace_bytes(int batch, int seqlen, int dim, int width);
void conv1d_bwd_workspace_layout(Conv1dBwdParams& q, void* workspace);

// ------------------------------------------------------------- widening helpers (widen.hip)
// dst[i0,i1,i2][tcol0 + c] = c < nvalid ? src[i0,i1,i2][scol0 + c] : 0   for c < ncols
// (element offsets: i0 * s0 + i1 * s1 + i2 * s2 for the source, t0..t2 for the destination).
struct ColCopy {
  int es;                      // element size: 2 (bf16) or 4 (fp32)
  int64_t d0, d1, d2, ncols, nvalid;
  const void* src; int64_t s0, s1, s2, scol0;
  void* dst; int64_t t0, t1, t2, tcol0;
};
hipError_t launch_col_copy(const ColCopy& c, hipStream_t st);
// dst[row][c] = (dst[row][c] + src[row][c]) * (gate ? silu(gate[row][c]) : 1), summed in fp32.
struct RowAdd {
  int es;
  int64_t d0, d1, d2, ncols;
  void* dst; int64_t t0, t1, t2;
  const void* src; int64_t s0, s1, s2;
  const void* gate; int64_t g0, g1, g2;
};
hipError_t launch_row_add(const RowAdd& a, hipStream_t st);
// The block's output gate: forward out = y silu(z); backward out = g silu(z), dz = g y silu'(z) (widen.hip).
struct GateParams {
  int es;
  int64_t d0, d1, d2, ncols;
  const void* y; int64_t y0, y1, y2;
  const void* z; int64_t z0, z1, z2;
  const void* g; int64_t g0, g1, g2;
  void* out; int64_t o0, o1, o2;
  void* dz; int64_t dz0, dz1, dz2;
};
hipError_t launch_gate(const GateParams& a, bool backward, hipStream_t st);

}  // namespace mh
