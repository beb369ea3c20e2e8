/*
 * mamformer_hip.h -- C ABI of libmamformer_hip.so, the MI355X (gfx950) scan path.
 *
 * The reference (Find-Vulnerabilities/Mamformer) has no FFI: its boundary is the
 * Python function API of the scan path.  Each entry point below replaces one of
 * those functions; the Python module mamformer_amd.ops binds them through
 * ctypes and keeps the reference names, argument order and layouts.
 * Paths are relative to "mamformer 671b/" in the reference tree.
 *
 * Conventions
 *  - All tensor pointers are device pointers owned by the caller; the library
 *    never allocates device memory at run time and never synchronises the
 *    stream (its one static device array, the scratch of
 *    mh_ssd_chunk_scan_fwd_noalloc, is created with the code object).
 *  - Strides are in elements.  The innermost dimension of every tensor is
 *    contiguous; 16-byte vector access requires 16-byte aligned base pointers
 *    and row strides that are multiples of 16 bytes (checked).
 *  - `stream` is a hipStream_t passed as void* (NULL = default stream).
 *  - Every call returns MH_OK (0) or a negative MH_ERR_* code; the detail of
 *    the last failure on the calling thread is returned by mh_last_error().
 *    Argument checks happen before any HIP call, so a rejected call has no
 *    side effect.
 */
#ifndef MAMFORMER_HIP_H
#define MAMFORMER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MH_ABI_VERSION 11

/* element types of x / B / C / y / q / k / v / o */
enum { MH_F32 = 0, MH_BF16 = 1 };

/* status codes */
enum {
  MH_OK = 0,
  MH_ERR_NULL = -1,        /* required pointer is NULL */
  MH_ERR_SHAPE = -2,       /* non-positive or inconsistent sizes */
  MH_ERR_DTYPE = -3,       /* unknown element type */
  MH_ERR_STRIDE = -4,      /* innermost dimension not contiguous / bad stride */
  MH_ERR_ALIGN = -5,       /* pointer or row stride not 16-byte aligned */
  MH_ERR_UNSUPPORTED = -6, /* size outside what the kernels implement */
  MH_ERR_WORKSPACE = -7,   /* workspace missing or too small */
  MH_ERR_HIP = -8          /* HIP launch error (message in mh_last_error) */
};

/* flags shared by the SSD entry points */
enum {
  MH_DT_SOFTPLUS = 1,      /* dt <- softplus(dt + dt_bias)   (mamba2.py:293, 304) */
  MH_DT_LIMIT = 2,         /* dt <- clamp(dt, dt_min, dt_max) after softplus */
  MH_D_PER_CHANNEL = 4,    /* D has nheads*headdim entries instead of nheads */
  MH_A_PER_STATE = 8,      /* decode only: A has dstate entries, one per state column (dA[p, n] = exp(A[n] dt)) */
  MH_DT_PER_CHANNEL = 16   /* decode only: dt (and dt_bias) have nheads*headdim entries, one per channel */
};

/* ------------------------------------------------------------------------
 * SSD chunked-scan prefill.
 * Replaces selective_scan / _selective_scan_impl
 *   (mamformer/layers/mamba2.py:31-67, 70-130) and triton_ssd_scan
 *   (mamformer/kernels/triton_ssd.py:508-564), in the per-head SSD convention:
 *   x (b, L, H, P), dt (b, L, H) fp32, A (H,) fp32 (A <= 0), B/C (b, L, G, N),
 *   D (H,) or (H*P,) fp32 or NULL, initial_state / final_state (b, H, P, N) fp32.
 *   y (b, L, H, P) in the dtype of x.  Supported: P = 64, N a multiple of 8 up to 256,
 *   H % G == 0.  chunk_len = state-passing chunk (multiple of 64; 0 = auto).
 *   The kernels tile N = 64 and 128; other N run as compositions of them (N < 64 zero-padded to 64,
 *   64 < N < 128 to 128, N > 128 as two 128-column halves whose outputs are summed), with B, C and
 *   the state pieces in the workspace.
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t batch, seqlen, nheads, headdim, dstate, ngroups;
  int64_t chunk_len;
  int32_t dtype;
  int32_t flags;
  float dt_min, dt_max;
  const void* x;   int64_t x_stride_b, x_stride_l, x_stride_h;
  const float* dt; int64_t dt_stride_b, dt_stride_l;
  const float* A;
  const void* B;   int64_t B_stride_b, B_stride_l;
  const void* C;   int64_t C_stride_b, C_stride_l;
  const float* D;
  const float* dt_bias;
  const float* initial_state;
  void* y;         int64_t y_stride_b, y_stride_l, y_stride_h;
  float* final_state;
  void* workspace; size_t workspace_bytes;
  /* optional output gate (NULL: none): y <- y * silu(z), z laid out like y in the dtype of x -- the
     z-gate that Mamba2Block.forward applies right after the scan (mamformer/layers/mamba2.py:337-338) */
  const void* z;   int64_t z_stride_b, z_stride_l, z_stride_h;
  /* optional (NULL: none), headdim 64: xsum (b, L, nheads, 2) fp32, the sums of x over each 32-channel half of a
     head per token.  mh_ssd_chunk_scan_fwd writes it (the scan has x on chip); mh_ssd_h_states and
     mh_ssd_h_states_bwd read it instead of x (h_states needs only these sums). */
  float* xsum;
} mh_ssd_args;

/* Bytes of workspace mh_ssd_chunk_scan_fwd needs for these sizes. */
int mh_ssd_workspace_bytes(const mh_ssd_args* a, size_t* bytes);
/* Resolved chunk_len (auto choice when a->chunk_len == 0). */
int mh_ssd_chunk_len(const mh_ssd_args* a, int64_t* chunk_len);
int mh_ssd_chunk_scan_fwd(const mh_ssd_args* a, void* stream);

/* Same prefill, allocating nothing: no counterpart in the reference.  For callers that cannot allocate
 *   device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 *   a->workspace / a->workspace_bytes are ignored: the kernels use a file-scope static device array of
 *   MH_NOALLOC_SCRATCH_BYTES, one per GPU the library runs on, held until the process ends.  Sizes whose
 *   workspace (mh_ssd_workspace_bytes) exceeds it are rejected with MH_ERR_WORKSPACE before any HIP
 *   call, and so is a dstate the kernels do not tile directly (anything but 64 and 128: those compositions
 *   need the caller's workspace), with MH_ERR_UNSUPPORTED.  Every call on one GPU uses that GPU's single array: calls that overlap in time on one GPU
 *   (several streams or host threads) race and must be serialised by the caller.  The first call on
 *   each GPU looks up the array's device address (hipGetSymbolAddress), which allocates nothing; make that
 *   first call outside stream capture (a capture may refuse the lookup), after which the entry point can be
 *   captured into a HIP graph and replayed (it records kernel launches only).
 *   Results are bit-identical to mh_ssd_chunk_scan_fwd's for the same arguments. */
#define MH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int mh_ssd_chunk_scan_fwd_noalloc(const mh_ssd_args* a, void* stream);

/* h_states of the prefill: hs (b, L, N) in the dtype of x, hs[b, t, n] = mean over (h, p) of the state after
 *   token t -- the h_states output of selective_scan / _selective_scan_impl (mamformer/layers/mamba2.py:114-116).
 *   Takes the forward's argument block (x, dt, A, B, dt flags, dt_bias, initial_state, workspace; y,
 *   final_state, C, D, z and chunk_len are not used) and computes the state's channel sums, which need one
 *   scalar per (token, head): sum_p x.  Supported: nheads <= 128, and the forward's dstate range. */
int mh_ssd_h_states_workspace_bytes(const mh_ssd_args* a, size_t* bytes);
int mh_ssd_h_states(const mh_ssd_args* a, void* h_states, void* stream);

/* The reference's own scan form: selective_scan / _selective_scan_impl (mamformer/layers/mamba2.py:31-130)
 *   literally, with a decay rate per state column and a step size per channel,
 *     h_t[c, n] = exp(A[n] dt_t[c]) h_{t-1}[c, n] + dt_t[c] x_t[c] B_t[n],  y_t[c] = sum_n C_t[n] h_t[c, n] + D[c] x_t[c]
 *   for the d_inner = nheads * headdim channels c (the caller passes A = -exp(clamp(A_log, -5, 5)), mamba2.py:87-90).
 *   Takes mh_ssd_args with flags MH_A_PER_STATE | MH_DT_PER_CHANNEL (required): A (dstate,) fp32; dt (b, L,
 *   d_inner) fp32 with dt_bias (d_inner,) and the softplus / limit flags as in the decode step; x, y and z (b, L,
 *   d_inner) with contiguous channels (x_stride_h = headdim); B, C (b, L, dstate) (ngroups 1); D (d_inner,) with
 *   MH_D_PER_CHANNEL or (nheads,) or NULL; initial_state / final_state (b, d_inner, dstate) fp32 or NULL (the
 *   reference starts from zero); chunk_len is ignored.  h_states (b, L, dstate) in the dtype of x, the mean over
 *   channels of the state after every token (mamba2.py:114-116), or NULL; it needs the workspace
 *   mh_ssd_ref_scan_workspace_bytes(a, 1, ..) gives (0 bytes without h_states).  Supported: dstate in {16, 32,
 *   64, 128, 256}, d_inner a multiple of 16.  Backward: mh_ssd_ref_scan_bwd below. */
int mh_ssd_ref_scan_workspace_bytes(const mh_ssd_args* a, int h_states, size_t* bytes);
int mh_ssd_ref_scan_fwd(const mh_ssd_args* a, void* h_states, void* stream);

/* Backward of the reference-form scan: the autograd backward of selective_scan / _selective_scan_impl in the
 *   reference's own parameterisation (mamformer/layers/mamba2.py:70-130, trained through in
 *   tests/test_mamba2.py:56-71), i.e. the gradients of <dy, y> + <dhs, h_states> + <d_final_state, final_state> for
 *   the call described by `fwd` (as mh_ssd_ref_scan_fwd reads it; fwd.y, final_state and workspace are ignored and
 *   fwd.z must be NULL: the gate's backward is mh_silu_gate_bwd).  dy, dx (b, L, d_inner) and dhs, dB, dC (b, L, N)
 *   contiguous in the dtype of x (dy, dhs NULL: zero); d_final_state, d_initial_state (b, d_inner, N) fp32 (NULL:
 *   zero / not wanted); ddt (b, L, d_inner) fp32 w.r.t. the raw dt (through dt_bias, softplus and the clamp); dA
 *   (N,) fp32 w.r.t. the rates A (the caller chains it to A_log through its clamp and exponential); dD like D;
 *   d_dt_bias (d_inner,) fp32.  Every output is overwritten; the sums over channels, tokens and batch rows are
 *   added in a fixed order (run-to-run identical).  The workspace holds the state at every 16th token (8th for
 *   dstate 256), b * ceil(L / 16) * d_inner * N fp32, and the channel-block partials. */
typedef struct {
  mh_ssd_args fwd;
  const void* dy;
  const void* dhs;
  const float* d_final_state;
  void* dx;
  float* ddt;
  float* dA;
  void* dB;
  void* dC;
  float* dD;
  float* d_dt_bias;
  float* d_initial_state;
  void* workspace; size_t workspace_bytes;
} mh_ssd_ref_bwd_args;
int mh_ssd_ref_scan_bwd_workspace_bytes(const mh_ssd_ref_bwd_args* a, size_t* bytes);
int mh_ssd_ref_scan_bwd(const mh_ssd_ref_bwd_args* a, void* stream);

/* Backward of h_states: the autograd backward of the mean over (h, p) of the states
 *   (mamformer/layers/mamba2.py:114-116) taken through the scan, i.e. the gradients of <dhs, h_states> for the
 *   call described by `fwd` (read as mh_ssd_h_states reads it).  dhs (b, L, N) contiguous in the dtype of x;
 *   dx (b, L, H, P) and dB (b, L, G, N) contiguous in the dtype of x; ddt (b, L, H) contiguous fp32 (w.r.t. the
 *   raw dt, through dt_bias, softplus and the clamp); dA (H,) fp32; d_dt_bias (H,) fp32 (required when
 *   fwd.dt_bias is set, else ignored); d_initial_state (b, H, P, N) fp32 or NULL.  Every output is overwritten
 *   (C, D and the gate get no gradient from h_states; the caller adds these to the output's gradients).
 *   dx_rows (optional): the gradient w.r.t. x is the same for every channel p of a (token, head); when dx_rows is
 *   set it is written there once per row, (b, L, H) fp32 contiguous, and dx is not written (may be NULL): pass it
 *   as mh_ssd_bwd_args.dx_rows of the scan's backward to have it added to the scan's dx on the way out.
 *   Supported: nheads <= 128, dstate <= 128. */
typedef struct {
  mh_ssd_args fwd;
  const void* dhs;
  void* dx;
  float* ddt;
  float* dA;
  void* dB;
  float* d_dt_bias;
  float* d_initial_state;
  void* workspace; size_t workspace_bytes;
  float* dx_rows;
} mh_ssd_hs_bwd_args;
int mh_ssd_h_states_bwd_workspace_bytes(const mh_ssd_hs_bwd_args* a, size_t* bytes);
int mh_ssd_h_states_bwd(const mh_ssd_hs_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------
 * SSD chunked-scan prefill backward.
 * Replaces the autograd backward of selective_scan / _selective_scan_impl
 *   (mamformer/layers/mamba2.py:70-130; trained through in tests/test_mamba2.py:56-71):
 *   gradients of <dy, y> + <d_final_state, final_state> for the forward call described by `fwd`
 *   (its x, dt, A, B, C, D, dt_bias, initial_state, flags, strides; fwd.y, fwd.final_state,
 *   fwd.workspace and fwd.chunk_len are ignored, fwd.z must be NULL and B/C may not broadcast).
 *   dy, dx (b, L, H, P) in the dtype of x; d_final_state, d_initial_state (b, H, P, N) fp32
 *   (NULL: zero / not wanted); ddt (b, L, H) fp32, the gradient w.r.t. the raw dt (through
 *   dt_bias, softplus and the clamp per fwd.flags); dA (H,) fp32; dB, dC (b, L, G, N) in the dtype
 *   of x; dD like D (NULL when D is NULL); d_dt_bias (H,) fp32 or NULL.  Every output is
 *   overwritten.  dx_rows (optional, NULL: none): (b, L, H) fp32 contiguous, added to every channel of
 *   dx[b, t, h, :] before it is stored (the h_states backward's dx_rows, so that the two gradients w.r.t. x
 *   meet without a second pass over dx).  Same supported sizes (and compositions) as the forward.
 * ---------------------------------------------------------------------- */
typedef struct {
  mh_ssd_args fwd;
  const void* dy;  int64_t dy_stride_b, dy_stride_l, dy_stride_h;
  const float* d_final_state;
  void* dx;        int64_t dx_stride_b, dx_stride_l, dx_stride_h;
  float* ddt;      int64_t ddt_stride_b, ddt_stride_l;
  float* dA;
  void* dB;        int64_t dB_stride_b, dB_stride_l;
  void* dC;        int64_t dC_stride_b, dC_stride_l;
  float* dD;
  float* d_dt_bias;
  float* d_initial_state;
  void* workspace; size_t workspace_bytes;
  const float* dx_rows;
} mh_ssd_bwd_args;

/* Bytes of workspace mh_ssd_chunk_scan_bwd needs for these sizes. */
int mh_ssd_bwd_workspace_bytes(const mh_ssd_bwd_args* a, size_t* bytes);
int mh_ssd_chunk_scan_bwd(const mh_ssd_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Single-token selective state update (decode step).
 * Replaces Mamba2Block._recurrent_step (mamformer/layers/mamba2.py:407-458):
 *   state (b, H, P, N) fp32 read from state_in and written to state_out (the
 *   two may alias: in-place update), x (b, H, P), dt (b, H) fp32 raw (bias,
 *   softplus and clamp applied per flags), A (H,), B/C (b, G, N), D, y (b, H, P).
 *   The reference's own parameterisation (a decay rate per state column, -exp(A_log) (N,), and a step
 *   size per channel, dt (b, d_inner), mamba2.py:440-446) is the flags MH_A_PER_STATE (A holds N
 *   entries) and MH_DT_PER_CHANNEL (dt and dt_bias hold H*P entries per row, d_inner = H*P).
 *   Supported: N in {8, 16, 32, 64, 128, 256}, H % G == 0.
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t batch, nheads, headdim, dstate, ngroups;
  int32_t dtype;
  int32_t flags;
  float dt_min, dt_max;
  const float* state_in;
  float* state_out;
  const void* x;   int64_t x_stride_b;
  const float* dt; int64_t dt_stride_b;
  const float* A;
  const void* B;   int64_t B_stride_b;
  const void* C;   int64_t C_stride_b;
  const float* D;
  const float* dt_bias;
  void* y;         int64_t y_stride_b;
  /* optional output gate (NULL: none): y <- y * silu(z), z (b, H, P) in the dtype of x
     (mamformer/layers/mamba2.py:337-338 on the one-token path) */
  const void* z;   int64_t z_stride_b;
} mh_ssu_args;

int mh_ssd_state_update(const mh_ssu_args* a, void* stream);

/* ------------------------------------------------------------------------
 * KDA linear-attention chunked scan, layout (B, H, S, D) contiguous.
 * mode MH_KDA_GATED: S_t = diag(exp(g_t)) S_{t-1} + k_t^T v_t,
 *                    o_t = q1_t S_t - lam q2_t S_t   (benchmark operator; no
 *                    reference function).  g (B,H,S,dk) fp32 or NULL (= 0).
 * mode MH_KDA_REFERENCE: the reference's phi(x) = elu(x)+1 normalised scan,
 *   replacing triton_linear_attn_scan (mamformer/kernels/triton_ssd.py:260-350)
 *   and LinearDiffAttention._linear_attention_scan
 *   (mamformer/layers/kda_diff.py:357-478): writes o1 and o2 separately.
 * initial_state / final_state (B,H,dk,dv) fp32 may be NULL.
 * Supported: dtype bf16 or fp32 (q, k, v, o share it), dk and dv each 64 or 128.  bf16 with
 *   dk = dv = 128 runs the bf16-MFMA kernels; every other combination runs kernels whose
 *   products are fp32 MFMA (fp32-accurate, for the fp32 I/O tolerance of 1e-4).
 * ---------------------------------------------------------------------- */
enum { MH_KDA_GATED = 0, MH_KDA_REFERENCE = 1 };

typedef struct {
  int64_t batch, nheads, seqlen, dk, dv;
  int32_t dtype;
  int32_t mode;
  int32_t kernel_dim;
  float lam;
  const float* lam_per_head;
  const void* q1; const void* q2; const void* k; const void* v;
  const float* g;
  const float* initial_state;
  const float* initial_z;
  float* final_state;
  float* final_z;
  void* o;
  void* o2;
} mh_kda_args;

int mh_kda_chunk_scan_fwd(const mh_kda_args* a, void* stream);

/* Backward of the reference-mode scan (fwd.mode == MH_KDA_REFERENCE): the
 *   gradient PyTorch autograd forms through LinearDiffAttention._linear_attention_scan
 *   (mamformer/layers/kda_diff.py:357-478) when the layer is trained.
 *   fwd: the forward's arguments (o, o2, final_state, final_z ignored).
 *   flags MH_KDA_BWD_DIFF: do1 is the gradient of the fused differential output
 *     (o1 - lam o2) / (1 - lam + 1e-8) (needs q2; lam from fwd.lam / lam_per_head)
 *     and d_lam (H,) fp32, if given, receives its gradient w.r.t. lam;
 *   otherwise do1 / do2 are the gradients of o1 / o2 (do2 NULL = zero).
 *   d_final_state (B,H,dk,dv) / d_final_z (B,H,dk) fp32: gradients of the final
 *   state and normaliser, or NULL (zero).
 *   Outputs dq1, dq2 (when q2), dk, dv (B,H,S,dk / dv) in the I/O dtype (zero beyond kernel_dim
 *   for dq, dk); d_initial_state / d_initial_z fp32 or NULL.
 *   Supported: as the forward (bf16 or fp32, dk and dv each 64 or 128).
 * ---------------------------------------------------------------------- */
enum { MH_KDA_BWD_DIFF = 1 };

typedef struct {
  mh_kda_args fwd;
  int32_t flags;
  const void* do1; const void* do2;
  const float* d_final_state; const float* d_final_z;
  void* dq1; void* dq2; void* dk; void* dv;
  float* d_initial_state; float* d_initial_z;
  float* d_lam;
  void* workspace; size_t workspace_bytes;
} mh_kda_bwd_args;

/* Bytes of workspace mh_kda_chunk_scan_bwd needs for these sizes. */
int mh_kda_bwd_workspace_bytes(const mh_kda_bwd_args* a, size_t* bytes);
int mh_kda_chunk_scan_bwd(const mh_kda_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------
 * One-token step of the reference-mode scan (KDA decode).
 * Replaces LinearDiffAttention._linear_attention_recurrent
 *   (mamformer/layers/kda_diff.py:564-605) together with the cache update of
 *   a one-token forward (kda_diff.py:329-338):
 *   S += phi(k)^T v, z += phi(k)  (state (B,H,dk,dv) fp32 and z (B,H,dk) fp32, in place),
 *   o_i = phi(q_i) S / (phi(q_i) z + 1e-8);  o = (o1 - lam o2) / (1 - lam + 1e-8) when o2 is NULL
 *   and q2 is given, else o = o1 (and o2 = o2 when given).
 *   q1/q2/k (B,H,dk), v/o/o2 (B,H,dv), contiguous.  flags: MH_KDA_PHI applies
 *   phi(x) = elu(x)+1 to the first kernel_dim channels of q/k (0 beyond); without
 *   it q/k are taken as already feature-mapped (the reference's calling form).
 *   Supported: dv in {64, 128, 256}, dk <= 16384 / dv.
 * ---------------------------------------------------------------------- */
enum { MH_KDA_PHI = 1 };

typedef struct {
  int64_t batch, nheads, dk, dv;
  int32_t dtype;
  int32_t flags;
  int32_t kernel_dim;
  float lam;
  const float* lam_per_head;
  const void* q1; const void* q2; const void* k; const void* v;
  float* state;
  float* z;
  void* o;
  void* o2;
} mh_kda_step_args;

int mh_kda_recurrent_step(const mh_kda_step_args* a, void* stream);

/* ------------------------------------------------------------------------
 * Causal depthwise conv1d (+ optional SiLU), the Mamba layer prologue.
 * Replaces Mamba2Block._causal_conv1d (mamformer/layers/mamba2.py:370-405)
 *   and the SiLU that follows it (mamba2.py:282-283):
 *   y[b,t,d] = act(bias[d] + sum_{j<width} weight[d,j] * xin[b, t-(width-1)+j, d])
 *   with xin = x for t >= 0, the last conv_state_len rows of conv_state
 *   (the cached raw inputs, mamba2.py:355-359) before that, and 0 beyond.
 *   x, conv_state, y (b, L, D) channels-last in one dtype, innermost
 *   contiguous; weight (D, width) fp32; bias (D,) fp32 or NULL.
 *   Supported: width 1..8, D % 8 == 0, conv_state_len <= width - 1.
 * ---------------------------------------------------------------------- */
enum { MH_CONV_SILU = 1 };

typedef struct {
  int64_t batch, seqlen, dim, width;
  int32_t dtype;
  int32_t flags;
  const void* x; int64_t x_stride_b, x_stride_l;
  const float* weight;
  const float* bias;
  const void* conv_state; int64_t conv_state_len, conv_state_stride_b, conv_state_stride_l;
  void* y; int64_t y_stride_b, y_stride_l;
} mh_conv1d_args;

int mh_causal_conv1d_fwd(const mh_conv1d_args* a, void* stream);

/* Backward of mh_causal_conv1d_fwd: the gradient PyTorch autograd forms through
 *   the reference's nn.Conv1d + F.silu (mamformer/layers/mamba2.py:279-283, :370-405)
 *   when Mamba2Block is trained (tests/test_mamba2.py:56-71).
 *   fwd: the forward's arguments (y ignored); dy (b, L, D) like x;
 *   dx (b, L, D) like x; d_conv_state (b, conv_state_len, D) like conv_state,
 *   the gradient of the cached rows (NULL: not computed); dweight (D, width)
 *   fp32 and dbias (D,) fp32 (or NULL) are overwritten with the sums over
 *   batch and tokens, deterministic (per 32-token-run partials reduced in a
 *   fixed order in the workspace).
 * ---------------------------------------------------------------------- */
typedef struct {
  mh_conv1d_args fwd;
  const void* dy; int64_t dy_stride_b, dy_stride_l;
  void* dx; int64_t dx_stride_b, dx_stride_l;
  void* d_conv_state; int64_t d_conv_state_stride_b, d_conv_state_stride_l;
  float* dweight;
  float* dbias;
  void* workspace; size_t workspace_bytes;
} mh_conv1d_bwd_args;

/* Bytes of workspace mh_causal_conv1d_bwd needs for these sizes. */
int mh_conv1d_bwd_workspace_bytes(const mh_conv1d_bwd_args* a, size_t* bytes);
int mh_causal_conv1d_bwd(const mh_conv1d_bwd_args* a, void* stream);

/* ------------------------------------------------------------------------ */
int mh_abi_version(void);
const char* mh_last_error(void);

/* ------------------------------------------------------------------------
 * The output gate of the Mamba-2 block, y * silu(z) (mamformer/layers/mamba2.py:337-338), for the training path,
 * where the ungated y is kept for the backward (the inference path gates inside the scan: mh_ssd_args.z).
 * Tensors (b, L, H, P) in `dtype` with innermost dimension contiguous and the other three strided (elements);
 * P a multiple of 8, 16-byte aligned rows.
 *   mh_silu_gate_fwd: out = y * silu(z).
 *   mh_silu_gate_bwd: with g the gradient of the gated output, dy = g * silu(z) and
 *                     dz = g * y * silu'(z), silu'(z) = s (1 + z (1 - s)), s = sigmoid(z); fp32 arithmetic.
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t batch, seqlen, nheads, headdim;
  int32_t dtype;
  int32_t reserved;
  const void* y;  int64_t y_stride_b, y_stride_l, y_stride_h;
  const void* z;  int64_t z_stride_b, z_stride_l, z_stride_h;
  const void* g;  int64_t g_stride_b, g_stride_l, g_stride_h;   /* backward only */
  void* out;      int64_t out_stride_b, out_stride_l, out_stride_h; /* forward: gated y; backward: dy */
  void* dz;       int64_t dz_stride_b, dz_stride_l, dz_stride_h;  /* backward only */
} mh_gate_args;
int mh_silu_gate_fwd(const mh_gate_args* a, void* stream);
int mh_silu_gate_bwd(const mh_gate_args* a, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MAMFORMER_HIP_H */
