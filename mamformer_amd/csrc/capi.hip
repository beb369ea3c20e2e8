// extern "C" entry points of libmamformer_hip.so (declared in include/mamformer_hip.h).
// Every entry point validates its argument block completely before the first
// HIP call, records a message for mh_last_error() on failure, then fills the
// internal parameter block and launches on the caller's stream.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "../../include/mamformer_hip.h"
#include "launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int elem_size(int32_t dtype) { return dtype == MH_F32 ? 4 : (dtype == MH_BF16 ? 2 : 0); }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
bool stride_ok(int64_t s, int es) { return s >= 0 && ((s * es) % 16) == 0; }

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MH_OK;
  return fail(MH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// ------------------------------------------------------------------ SSD prefill
constexpr int64_t kMaxDim = (int64_t)1 << 30;

int ssd_heads_per_wg(const mh_ssd_args* a) {
  const int64_t hpg = a->nheads / a->ngroups;
  // fp32 tiles with N = 128 are twice the bf16 size: one head per workgroup
  // keeps the running state and operands in registers.
  const int64_t n = a->dstate <= 64 ? 64 : 128;                 // dstate the kernels run
  int hg = (a->dtype == MH_F32 && n == 128) ? 1 : 4;
  while (hg > 1 && (hpg % hg) != 0) hg >>= 1;
  return hg;
}

int64_t ssd_auto_chunk(const mh_ssd_args* a) {
  const int64_t hg = ssd_heads_per_wg(a);
  const int64_t units = a->batch * (a->nheads / hg);           // workgroups per chunk index
  const int64_t target = 256;                                   // one 8-wave workgroup per CU on 256 CUs
  int64_t want = (a->seqlen * units + target - 1) / target;     // tokens per workgroup
  want = ((want + 63) / 64) * 64;
  if (want < 256) want = 256;
  if (want > 16384) want = 16384;
  return want;
}

int ssd_validate(const mh_ssd_args* a, int64_t* chunk_len_out) {
  if (!a) return fail(MH_ERR_NULL, "ssd: args is NULL");
  if (a->batch <= 0 || a->seqlen < 0 || a->nheads <= 0 || a->headdim <= 0 || a->dstate <= 0 || a->ngroups <= 0)
    return fail(MH_ERR_SHAPE, "ssd: sizes must be positive (batch=%lld seqlen=%lld nheads=%lld headdim=%lld dstate=%lld ngroups=%lld)",
                (long long)a->batch, (long long)a->seqlen, (long long)a->nheads, (long long)a->headdim,
                (long long)a->dstate, (long long)a->ngroups);
  if (a->batch > kMaxDim || a->seqlen > kMaxDim || a->nheads > 65535)
    return fail(MH_ERR_SHAPE, "ssd: sizes out of range");
  if (a->nheads % a->ngroups)
    return fail(MH_ERR_SHAPE, "ssd: nheads (%lld) must be a multiple of ngroups (%lld)", (long long)a->nheads,
                (long long)a->ngroups);
  const int es = elem_size(a->dtype);
  if (!es) return fail(MH_ERR_DTYPE, "ssd: unknown dtype %d", a->dtype);
  if (a->headdim != 64) return fail(MH_ERR_UNSUPPORTED, "ssd: headdim %lld not supported (64)", (long long)a->headdim);
  if (a->dstate % 8 || a->dstate > 256)
    return fail(MH_ERR_UNSUPPORTED, "ssd: dstate %lld not supported (a multiple of 8 up to 256)", (long long)a->dstate);
  int64_t cl = a->chunk_len;
  if (cl == 0) cl = ssd_auto_chunk(a);
  if (cl < 64 || cl % 64 || cl > (1 << 20))
    return fail(MH_ERR_SHAPE, "ssd: chunk_len %lld must be a positive multiple of 64", (long long)a->chunk_len);
  if ((a->flags & MH_DT_LIMIT) && !(a->dt_min <= a->dt_max))
    return fail(MH_ERR_SHAPE, "ssd: dt_min > dt_max");
  if (a->flags & (MH_A_PER_STATE | MH_DT_PER_CHANNEL))
    return fail(MH_ERR_UNSUPPORTED, "ssd: MH_A_PER_STATE / MH_DT_PER_CHANNEL are decode-step flags (the chunked "
                                    "scan factorises a per-head decay)");
  if (!a->A) return fail(MH_ERR_NULL, "ssd: A is required");
  if (a->seqlen > 0 && (!a->x || !a->dt || !a->B || !a->C || !a->y))
    return fail(MH_ERR_NULL, "ssd: x, dt, A, B, C, y are required");
  if (!aligned16(a->x) || !aligned16(a->B) || !aligned16(a->C) || !aligned16(a->y))
    return fail(MH_ERR_ALIGN, "ssd: x, B, C, y must be 16-byte aligned");
  if (!stride_ok(a->x_stride_b, es) || !stride_ok(a->x_stride_l, es) || !stride_ok(a->x_stride_h, es) ||
      !stride_ok(a->y_stride_b, es) || !stride_ok(a->y_stride_l, es) || !stride_ok(a->y_stride_h, es) ||
      !stride_ok(a->B_stride_b, es) || !stride_ok(a->B_stride_l, es) || !stride_ok(a->C_stride_b, es) ||
      !stride_ok(a->C_stride_l, es))
    return fail(MH_ERR_ALIGN, "ssd: strides of x, y, B, C must be multiples of 16 bytes");
  if (a->dt_stride_b < 0 || a->dt_stride_l < 0) return fail(MH_ERR_STRIDE, "ssd: negative dt stride");
  // the kernels address one 64-token segment of x / y / B / C / dt with 32-bit offsets
  constexpr int64_t kSpan = (int64_t)1 << 31;
  if (a->x_stride_l * es * 64 >= kSpan || a->y_stride_l * es * 64 >= kSpan || a->B_stride_l * es * 64 >= kSpan ||
      a->C_stride_l * es * 64 >= kSpan || a->dt_stride_l * 4 * 64 >= kSpan)
    return fail(MH_ERR_STRIDE, "ssd: token stride too large (64 tokens must span less than 2 GiB)");
  if (a->x_stride_h < a->headdim || a->y_stride_h < a->headdim)
    return fail(MH_ERR_STRIDE, "ssd: x/y head stride smaller than headdim (headdim must be contiguous)");
  if (a->z) {
    if (!aligned16(a->z)) return fail(MH_ERR_ALIGN, "ssd: z must be 16-byte aligned");
    if (!stride_ok(a->z_stride_b, es) || !stride_ok(a->z_stride_l, es) || !stride_ok(a->z_stride_h, es))
      return fail(MH_ERR_ALIGN, "ssd: strides of z must be multiples of 16 bytes");
    if (a->z_stride_h < a->headdim)
      return fail(MH_ERR_STRIDE, "ssd: z head stride smaller than headdim (headdim must be contiguous)");
    if (a->z_stride_l * es * 64 >= ((int64_t)1 << 31))
      return fail(MH_ERR_STRIDE, "ssd: z token stride too large (64 tokens must span less than 2 GiB)");
  }
  if (a->xsum && !aligned16(a->xsum)) return fail(MH_ERR_ALIGN, "ssd: xsum must be 16-byte aligned");
  if ((a->B_stride_l != 0 && a->B_stride_l < a->ngroups * a->dstate) ||
      (a->C_stride_l != 0 && a->C_stride_l < a->ngroups * a->dstate))
    return fail(MH_ERR_STRIDE, "ssd: B/C token stride smaller than ngroups*dstate ((g, n) must be contiguous; 0 broadcasts)");
  const int64_t nchunks = (a->seqlen + cl - 1) / cl;
  if (nchunks > 65535) return fail(MH_ERR_SHAPE, "ssd: too many chunks (%lld)", (long long)nchunks);
  if (chunk_len_out) *chunk_len_out = cl;
  return MH_OK;
}

// ------------------------------------------------------------------ decode
int ssu_validate(const mh_ssu_args* a) {
  if (!a) return fail(MH_ERR_NULL, "state_update: args is NULL");
  if (a->batch <= 0 || a->nheads <= 0 || a->headdim <= 0 || a->dstate <= 0 || a->ngroups <= 0)
    return fail(MH_ERR_SHAPE, "state_update: sizes must be positive");
  if (a->batch * a->nheads > 0x7fffffffLL || a->headdim > 4096)
    return fail(MH_ERR_SHAPE, "state_update: sizes out of range");
  if (a->nheads % a->ngroups) return fail(MH_ERR_SHAPE, "state_update: nheads must be a multiple of ngroups");
  const int es = elem_size(a->dtype);
  if (!es) return fail(MH_ERR_DTYPE, "state_update: unknown dtype %d", a->dtype);
  switch (a->dstate) {
    case 8: case 16: case 32: case 64: case 128: case 256: break;
    default: return fail(MH_ERR_UNSUPPORTED, "state_update: dstate %lld not supported (8..256, power of two)",
                         (long long)a->dstate);
  }
  if ((a->flags & MH_DT_LIMIT) && !(a->dt_min <= a->dt_max)) return fail(MH_ERR_SHAPE, "state_update: dt_min > dt_max");
  if (!a->state_in || !a->state_out || !a->x || !a->dt || !a->A || !a->B || !a->C || !a->y)
    return fail(MH_ERR_NULL, "state_update: state_in, state_out, x, dt, A, B, C, y are required");
  if (!aligned16(a->state_in) || !aligned16(a->state_out))
    return fail(MH_ERR_ALIGN, "state_update: state must be 16-byte aligned");
  if (a->z && a->z_stride_b < a->nheads * a->headdim)
    return fail(MH_ERR_STRIDE, "state_update: z batch stride smaller than a row ((h, p) contiguous)");
  if (a->x_stride_b < a->nheads * a->headdim || a->y_stride_b < a->nheads * a->headdim ||
      a->B_stride_b < a->ngroups * a->dstate || a->C_stride_b < a->ngroups * a->dstate ||
      a->dt_stride_b < ((a->flags & MH_DT_PER_CHANNEL) ? a->nheads * a->headdim : a->nheads))
    return fail(MH_ERR_STRIDE, "state_update: batch stride smaller than a row ((h, p) / (g, n) / h contiguous)");
  if (a->state_in != a->state_out) {
    const uintptr_t bytes = (uintptr_t)(a->batch * a->nheads * a->headdim * a->dstate * 4);
    const uintptr_t i0 = (uintptr_t)a->state_in, o0 = (uintptr_t)a->state_out;
    if (i0 < o0 + bytes && o0 < i0 + bytes)
      return fail(MH_ERR_STRIDE, "state_update: state_in and state_out overlap without being identical");
  }
  return MH_OK;
}

// ------------------------------------------------------------------ KDA
int kda_validate(const mh_kda_args* a) {
  if (!a) return fail(MH_ERR_NULL, "kda: args is NULL");
  if (a->batch <= 0 || a->nheads <= 0 || a->seqlen < 0 || a->dk <= 0 || a->dv <= 0)
    return fail(MH_ERR_SHAPE, "kda: sizes must be positive");
  if (a->batch * a->nheads > 0x7fffffffLL || a->seqlen > kMaxDim) return fail(MH_ERR_SHAPE, "kda: sizes out of range");
  if (!elem_size(a->dtype)) return fail(MH_ERR_DTYPE, "kda: unknown dtype %d", a->dtype);
  if (a->mode != MH_KDA_GATED && a->mode != MH_KDA_REFERENCE) return fail(MH_ERR_UNSUPPORTED, "kda: unknown mode %d", a->mode);
  if ((a->dk != 64 && a->dk != 128) || (a->dv != 64 && a->dv != 128))
    return fail(MH_ERR_UNSUPPORTED, "kda: dk=%lld dv=%lld not supported (each 64 or 128)", (long long)a->dk,
                (long long)a->dv);
  if (a->seqlen > 0 && (!a->q1 || !a->k || !a->v || !a->o))
    return fail(MH_ERR_NULL, "kda: q1, k, v, o are required");
  if (a->mode == MH_KDA_REFERENCE) {
    if (a->kernel_dim <= 0) return fail(MH_ERR_SHAPE, "kda: kernel_dim must be positive");
    if (a->g) return fail(MH_ERR_SHAPE, "kda: reference mode takes no gate g");
    if (!a->q2 && a->o2) return fail(MH_ERR_NULL, "kda: o2 given without q2");
  } else {
    if (a->o2 || a->initial_z || a->final_z) return fail(MH_ERR_SHAPE, "kda: o2 / initial_z / final_z are reference-mode outputs");
  }
  if (!aligned16(a->q1) || (a->q2 && !aligned16(a->q2)) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o) ||
      (a->o2 && !aligned16(a->o2)) || (a->g && !aligned16(a->g)))
    return fail(MH_ERR_ALIGN, "kda: tensors must be 16-byte aligned");
  return MH_OK;
}

int kda_step_validate(const mh_kda_step_args* a) {
  if (!a) return fail(MH_ERR_NULL, "kda_step: args is NULL");
  if (a->batch <= 0 || a->nheads <= 0 || a->dk <= 0 || a->dv <= 0) return fail(MH_ERR_SHAPE, "kda_step: sizes must be positive");
  if (a->batch * a->nheads > 0x7fffffffLL) return fail(MH_ERR_SHAPE, "kda_step: sizes out of range");
  if (!elem_size(a->dtype)) return fail(MH_ERR_DTYPE, "kda_step: unknown dtype %d", a->dtype);
  if (a->dv != 64 && a->dv != 128 && a->dv != 256)
    return fail(MH_ERR_UNSUPPORTED, "kda_step: dv %lld not supported (64, 128, 256)", (long long)a->dv);
  if (a->dk > 16384 / a->dv) return fail(MH_ERR_UNSUPPORTED, "kda_step: dk %lld > %lld", (long long)a->dk, (long long)(16384 / a->dv));
  if ((a->flags & MH_KDA_PHI) && a->kernel_dim <= 0) return fail(MH_ERR_SHAPE, "kda_step: kernel_dim must be positive");
  if (!a->q1 || !a->k || !a->v || !a->state || !a->z || !a->o)
    return fail(MH_ERR_NULL, "kda_step: q1, k, v, state, z, o are required");
  if (!a->q2 && a->o2) return fail(MH_ERR_NULL, "kda_step: o2 given without q2");
  if (!aligned16(a->state)) return fail(MH_ERR_ALIGN, "kda_step: state must be 16-byte aligned");
  return MH_OK;
}

int conv_validate(const mh_conv1d_args* a) {
  if (!a) return fail(MH_ERR_NULL, "conv1d: args is NULL");
  if (a->batch <= 0 || a->seqlen < 0 || a->dim <= 0 || a->width <= 0)
    return fail(MH_ERR_SHAPE, "conv1d: sizes must be positive");
  if (a->batch > 65535 || a->seqlen > kMaxDim || a->dim > kMaxDim) return fail(MH_ERR_SHAPE, "conv1d: sizes out of range");
  if (a->width > 8) return fail(MH_ERR_UNSUPPORTED, "conv1d: width %lld not supported (1..8)", (long long)a->width);
  if (a->dim % 8) return fail(MH_ERR_UNSUPPORTED, "conv1d: dim %lld must be a multiple of 8", (long long)a->dim);
  const int es = elem_size(a->dtype);
  if (!es) return fail(MH_ERR_DTYPE, "conv1d: unknown dtype %d", a->dtype);
  if (!a->weight) return fail(MH_ERR_NULL, "conv1d: weight is required");
  if (a->seqlen > 0 && (!a->x || !a->y)) return fail(MH_ERR_NULL, "conv1d: x and y are required");
  if (a->conv_state_len < 0 || a->conv_state_len > a->width - 1)
    return fail(MH_ERR_SHAPE, "conv1d: conv_state_len %lld outside [0, width-1]", (long long)a->conv_state_len);
  if (a->conv_state_len > 0 && !a->conv_state) return fail(MH_ERR_NULL, "conv1d: conv_state is NULL");
  if (!aligned16(a->x) || !aligned16(a->y) || (a->conv_state && !aligned16(a->conv_state)))
    return fail(MH_ERR_ALIGN, "conv1d: x, y, conv_state must be 16-byte aligned");
  if (!stride_ok(a->x_stride_b, es) || !stride_ok(a->x_stride_l, es) || !stride_ok(a->y_stride_b, es) ||
      !stride_ok(a->y_stride_l, es) ||
      (a->conv_state && (!stride_ok(a->conv_state_stride_b, es) || !stride_ok(a->conv_state_stride_l, es))))
    return fail(MH_ERR_ALIGN, "conv1d: strides must be multiples of 16 bytes");
  if (a->x_stride_l < a->dim || a->y_stride_l < a->dim)
    return fail(MH_ERR_STRIDE, "conv1d: token stride smaller than dim (channels must be contiguous)");
  return MH_OK;
}

// ------------------------------------------------------------------ static scratch (no-allocation entry)
// The workspace of mh_ssd_chunk_scan_fwd_noalloc: one array per GPU, created with the code object and held
// until the process ends.  Host code never passes `scratch` itself to a kernel (its host-side name is not a
// device address); it uses the per-device address hipGetSymbolAddress returns, looked up once per device.
__device__ __align__(256) unsigned char scratch[MH_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxDevices] = {};

// Device address of `scratch` on the device `stream` belongs to (the current device for the null stream).
int scratch_address(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice(stream, &dev);
  if (e != hipSuccess) return hip_status(e, "ssd_noalloc: hipStreamGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(MH_ERR_UNSUPPORTED, "ssd_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_status(e, "ssd_noalloc: hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_status(e, "ssd_noalloc: hipSetDevice");
    void* addr = nullptr;
    const hipError_t es = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (cur != dev && (e = hipSetDevice(cur)) != hipSuccess) return hip_status(e, "ssd_noalloc: hipSetDevice");
    if (es != hipSuccess) return hip_status(es, "ssd_noalloc: hipGetSymbolAddress(scratch)");
    if (!addr) return fail(MH_ERR_HIP, "ssd_noalloc: hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_addr[dev] = addr;
  }
  *out = g_scratch_addr[dev];
  return MH_OK;
}

// Forward parameter block from a validated argument struct (workspace not laid out).
void ssd_fill(const mh_ssd_args* a, int64_t cl, int64_t nchunks, mh::SsdParams& p) {
  memset(&p, 0, sizeof(p));
  p.batch = (int)a->batch; p.seqlen = (int)a->seqlen; p.nheads = (int)a->nheads; p.headdim = (int)a->headdim;
  p.dstate = (int)a->dstate; p.ngroups = (int)a->ngroups; p.dtype = a->dtype;
  p.chunk_len = (int)cl; p.nchunks = (int)nchunks; p.heads_per_wg = ssd_heads_per_wg(a);
  p.dt_softplus = (a->flags & MH_DT_SOFTPLUS) != 0;
  p.has_dt_limit = (a->flags & MH_DT_LIMIT) != 0;
  p.D_per_channel = (a->flags & MH_D_PER_CHANNEL) != 0;
  p.dt_min = a->dt_min; p.dt_max = a->dt_max;
  p.x = a->x; p.x_sb = a->x_stride_b; p.x_sl = a->x_stride_l; p.x_sh = a->x_stride_h;
  p.dt = a->dt; p.dt_sb = a->dt_stride_b; p.dt_sl = a->dt_stride_l;
  p.A = a->A;
  p.B = a->B; p.B_sb = a->B_stride_b; p.B_sl = a->B_stride_l;
  p.C = a->C; p.C_sb = a->C_stride_b; p.C_sl = a->C_stride_l;
  p.D = a->D; p.dt_bias = a->dt_bias; p.init_state = a->initial_state;
  p.y = a->y; p.y_sb = a->y_stride_b; p.y_sl = a->y_stride_l; p.y_sh = a->y_stride_h;
  p.final_state = a->final_state;
  p.z = a->z; p.z_sb = a->z_stride_b; p.z_sl = a->z_stride_l; p.z_sh = a->z_stride_h;
  p.nseg = (int)((a->seqlen + 63) / 64);
  p.xsum = a->xsum;
}

int ssd_bwd_validate(const mh_ssd_bwd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "ssd_bwd: args is NULL");
  const mh_ssd_args* f = &a->fwd;
  if (f->z) return fail(MH_ERR_UNSUPPORTED, "ssd_bwd: the output gate is not differentiated here (fwd.z must be NULL)");
  // the forward's checks, with the outputs the backward does not touch taken from x and 64-token chunks
  mh_ssd_args g = *f;
  g.y = const_cast<void*>(g.x); g.y_stride_b = g.x_stride_b; g.y_stride_l = g.x_stride_l; g.y_stride_h = g.x_stride_h;
  g.chunk_len = 64;
  int rc = ssd_validate(&g, nullptr);
  if (rc) return rc;
  const int es = elem_size(f->dtype);
  if (f->seqlen > 0 && (f->B_stride_l == 0 || f->C_stride_l == 0))
    return fail(MH_ERR_UNSUPPORTED, "ssd_bwd: broadcast B/C (token stride 0) not supported");
  if (f->seqlen > 0 && (!a->dy || !a->dx || !a->ddt || !a->dB || !a->dC))
    return fail(MH_ERR_NULL, "ssd_bwd: dy, dx, ddt, dB, dC are required");
  if (!a->dA) return fail(MH_ERR_NULL, "ssd_bwd: dA is required");
  if (f->D && !a->dD) return fail(MH_ERR_NULL, "ssd_bwd: dD is required when D is given");
  if (!aligned16(a->dy) || !aligned16(a->dx) || !aligned16(a->dB) || !aligned16(a->dC) ||
      !aligned16(a->d_final_state) || !aligned16(a->d_initial_state))
    return fail(MH_ERR_ALIGN, "ssd_bwd: dy, dx, dB, dC, d_final_state, d_initial_state must be 16-byte aligned");
  if (!stride_ok(a->dy_stride_b, es) || !stride_ok(a->dy_stride_l, es) || !stride_ok(a->dy_stride_h, es) ||
      !stride_ok(a->dx_stride_b, es) || !stride_ok(a->dx_stride_l, es) || !stride_ok(a->dx_stride_h, es) ||
      !stride_ok(a->dB_stride_b, es) || !stride_ok(a->dB_stride_l, es) || !stride_ok(a->dC_stride_b, es) ||
      !stride_ok(a->dC_stride_l, es))
    return fail(MH_ERR_ALIGN, "ssd_bwd: strides of dy, dx, dB, dC must be multiples of 16 bytes");
  if (a->dy_stride_h < f->headdim || a->dx_stride_h < f->headdim)
    return fail(MH_ERR_STRIDE, "ssd_bwd: dy/dx head stride smaller than headdim (headdim must be contiguous)");
  if (reinterpret_cast<uintptr_t>(a->dx_rows) % 4) return fail(MH_ERR_ALIGN, "ssd_bwd: dx_rows must be 4-byte aligned");
  if (a->dB_stride_l < f->ngroups * f->dstate || a->dC_stride_l < f->ngroups * f->dstate)
    return fail(MH_ERR_STRIDE, "ssd_bwd: dB/dC token stride smaller than ngroups*dstate");
  if (a->ddt_stride_b < 0 || a->ddt_stride_l < 0) return fail(MH_ERR_STRIDE, "ssd_bwd: negative ddt stride");
  constexpr int64_t kSpan = (int64_t)1 << 31;
  if (a->dy_stride_l * es * 64 >= kSpan)
    return fail(MH_ERR_STRIDE, "ssd_bwd: dy token stride too large (64 tokens must span less than 2 GiB)");
  return MH_OK;
}

// Heads of one group per workgroup of the gradient kernel: the largest of 16, 8, 4, 2, 1 dividing H / G.
int ssd_bwd_heads_per_wg(const mh_ssd_args* f) {
  const int64_t hpg = f->nheads / f->ngroups;
  int hb = 16;
  while (hb > 1 && hpg % hb) hb >>= 1;
  return hb;
}

hipError_t ssd_launch_bwd_native(const mh_ssd_bwd_args* a, hipStream_t st) {
  const mh_ssd_args* f = &a->fwd;
  mh::SsdBwdParams q;
  memset(&q, 0, sizeof(q));
  const int64_t nseg = (f->seqlen + 63) / 64;
  ssd_fill(f, 64, nseg, q.f);
  q.f.y = nullptr;
  q.f.final_state = nullptr;
  q.f.z = nullptr;
  q.dy = a->dy; q.dy_sb = a->dy_stride_b; q.dy_sl = a->dy_stride_l; q.dy_sh = a->dy_stride_h;
  q.d_final = a->d_final_state;
  q.dx = a->dx; q.dx_sb = a->dx_stride_b; q.dx_sl = a->dx_stride_l; q.dx_sh = a->dx_stride_h;
  q.ddt = a->ddt; q.ddt_sb = a->ddt_stride_b; q.ddt_sl = a->ddt_stride_l;
  q.dA = a->dA; q.dD = f->D ? a->dD : nullptr; q.dbias = a->d_dt_bias; q.dh0 = a->d_initial_state;
  q.dB = a->dB; q.dB_sb = a->dB_stride_b; q.dB_sl = a->dB_stride_l;
  q.dC = a->dC; q.dC_sb = a->dC_stride_b; q.dC_sl = a->dC_stride_l;
  q.heads_per_wg = ssd_bwd_heads_per_wg(f);
  q.dx_rows = a->dx_rows;
  if (nseg > 0) mh::ssd_bwd_workspace_layout(q, a->workspace);
  return mh::launch_ssd_bwd(q, st);
}

// ------------------------------------------------------------------ SSD state sizes by composition
// The prefill and backward kernels tile dstate 64 and 128.  Other sizes (multiples of 8 up to 256) run as
// compositions: up to 64 zero-padded at 64, up to 128 zero-padded at 128, above 128 as two runs over the
// 128-column halves of B, C and the state, the second half zero-padded (widen.hip states why these are
// exact); the pieces of B, C and the states pass through the workspace.
bool ssd_native_dstate(int64_t n) { return n == 64 || n == 128; }
int64_t ssd_inner_dstate(int64_t n) { return n <= 64 ? 64 : 128; }
size_t a256(size_t x) { return (x + 255) & ~(size_t)255; }
char* at(void* base, size_t off) { return reinterpret_cast<char*>(base) + off; }

struct SsdWide {
  int64_t ni;              // dstate of the inner runs
  int pieces;              // 1 (padded) or 2 (halves)
  bool copy_bc;            // B / C (and dB / dC) pieces pass through the workspace
  size_t inner;            // workspace of one inner run (at offset 0)
  size_t oB, oC, oS0, oS1, oX2, oT2, oH2, oH3, total;
};

// Forward: oS0 = initial-state piece, oS1 = final-state piece, oX2 = y of the second half.
void ssd_wide_fwd_plan(const mh_ssd_args* a, int64_t cl, SsdWide& w) {
  const int es = elem_size(a->dtype);
  const int64_t b = a->batch, L = a->seqlen, H = a->nheads, P = a->headdim, G = a->ngroups;
  w.ni = ssd_inner_dstate(a->dstate);
  w.pieces = a->dstate > 128 ? 2 : 1;
  w.copy_bc = a->dstate != w.pieces * w.ni || G > 1;
  const int64_t nchunks = (L + cl - 1) / cl;
  w.inner = nchunks > 0 ? mh::ssd_workspace_bytes((int)b, (int)L, (int)nchunks, (int)H, (int)P, (int)w.ni, (int)G,
                                                  a->dtype) : 0;
  const size_t bc = w.copy_bc ? (size_t)(b * L * G * w.ni * es) : 0, st = (size_t)(b * H * P * w.ni * 4);
  size_t off = a256(w.inner);
  w.oB = off; off += a256(bc);
  w.oC = off; off += a256(bc);
  w.oS0 = off; off += a->initial_state ? a256(st) : 0;
  w.oS1 = off; off += a->final_state ? a256(st) : 0;
  w.oX2 = off; off += w.pieces == 2 ? a256((size_t)(b * L * H * P * es)) : 0;
  w.oT2 = w.oH2 = w.oH3 = off;
  w.total = off;
}

// Column piece q of a (b, L, G, N) B/C-shaped tensor into a (b, L, G, ni) workspace buffer (zero-padded), or back.
mh::ColCopy bc_in(const mh_ssd_args* a, const void* src, int64_t sb, int64_t sl, void* dst, int64_t ni, int q) {
  mh::ColCopy c{};
  c.es = elem_size(a->dtype);
  c.d0 = a->batch; c.d1 = a->seqlen; c.d2 = a->ngroups;
  c.ncols = ni; c.nvalid = std::min<int64_t>(ni, a->dstate - q * ni);
  c.src = src; c.s0 = sb; c.s1 = sl; c.s2 = a->dstate; c.scol0 = q * ni;
  c.dst = dst; c.t2 = ni; c.t1 = a->ngroups * ni; c.t0 = a->seqlen * c.t1; c.tcol0 = 0;
  return c;
}
mh::ColCopy bc_out(const mh_ssd_args* a, const void* src, void* dst, int64_t tb, int64_t tl, int64_t ni, int q) {
  mh::ColCopy c{};
  c.es = elem_size(a->dtype);
  c.d0 = a->batch; c.d1 = a->seqlen; c.d2 = a->ngroups;
  c.ncols = c.nvalid = std::min<int64_t>(ni, a->dstate - q * ni);
  c.src = src; c.s2 = ni; c.s1 = a->ngroups * ni; c.s0 = a->seqlen * c.s1; c.scol0 = 0;
  c.dst = dst; c.t0 = tb; c.t1 = tl; c.t2 = a->dstate; c.tcol0 = q * ni;
  return c;
}
// Column piece q of a (b, H, P, N) fp32 state into a (b, H, P, ni) buffer (zero-padded), or back.
mh::ColCopy state_in(const mh_ssd_args* a, const float* src, void* dst, int64_t ni, int q) {
  mh::ColCopy c{};
  c.es = 4;
  c.d0 = a->batch; c.d1 = a->nheads; c.d2 = a->headdim;
  c.ncols = ni; c.nvalid = std::min<int64_t>(ni, a->dstate - q * ni);
  c.src = src; c.s2 = a->dstate; c.s1 = a->headdim * c.s2; c.s0 = a->nheads * c.s1; c.scol0 = q * ni;
  c.dst = dst; c.t2 = ni; c.t1 = a->headdim * ni; c.t0 = a->nheads * c.t1; c.tcol0 = 0;
  return c;
}
mh::ColCopy state_out(const mh_ssd_args* a, const void* src, float* dst, int64_t ni, int q) {
  mh::ColCopy c{};
  c.es = 4;
  c.d0 = a->batch; c.d1 = a->nheads; c.d2 = a->headdim;
  c.ncols = c.nvalid = std::min<int64_t>(ni, a->dstate - q * ni);
  c.src = src; c.s2 = ni; c.s1 = a->headdim * ni; c.s0 = a->nheads * c.s1; c.scol0 = 0;
  c.dst = dst; c.t2 = a->dstate; c.t1 = a->headdim * c.t2; c.t0 = a->nheads * c.t1; c.tcol0 = q * ni;
  return c;
}

// The inner forward arguments of piece q (B, C, D and the state pointers set; outputs by the caller).
mh_ssd_args ssd_piece(const mh_ssd_args* a, const SsdWide& w, void* ws, int q) {
  const int es = elem_size(a->dtype);
  mh_ssd_args in = *a;
  in.dstate = w.ni;
  if (w.copy_bc) {
    in.B = at(ws, w.oB); in.C = at(ws, w.oC);
    in.B_stride_l = in.C_stride_l = a->ngroups * w.ni;
    in.B_stride_b = in.C_stride_b = a->seqlen * a->ngroups * w.ni;
  } else {                 // one group: the half is a column offset with the caller's strides
    in.B = reinterpret_cast<const char*>(a->B) + q * w.ni * es;
    in.C = reinterpret_cast<const char*>(a->C) + q * w.ni * es;
  }
  if (q > 0) { in.D = nullptr; in.flags &= ~MH_D_PER_CHANNEL; }    // D x enters y once
  in.initial_state = a->initial_state ? reinterpret_cast<const float*>(at(ws, w.oS0)) : nullptr;
  in.final_state = nullptr;
  in.z = nullptr;
  in.workspace = ws; in.workspace_bytes = w.inner;
  return in;
}

hipError_t ssd_launch_native(const mh_ssd_args* a, int64_t cl, void* ws, hipStream_t st) {
  const int64_t nchunks = (a->seqlen + cl - 1) / cl;
  mh::SsdParams p;
  ssd_fill(a, cl, nchunks, p);
  if (nchunks > 0) mh::ssd_workspace_layout(p, ws);
  return mh::launch_ssd(p, st);
}

int ssd_fwd_wide(const mh_ssd_args* a, int64_t cl, hipStream_t st) {
  SsdWide w;
  ssd_wide_fwd_plan(a, cl, w);
  void* ws = a->workspace;
  const int es = elem_size(a->dtype);
  const int64_t b = a->batch, L = a->seqlen, H = a->nheads, P = a->headdim;
  hipError_t e = hipSuccess;
  for (int q = 0; q < w.pieces && e == hipSuccess; ++q) {
    mh_ssd_args in = ssd_piece(a, w, ws, q);
    in.chunk_len = cl;
    if (q == 0) {
      in.y = a->y;
      if (w.pieces == 1) in.z = a->z;
    } else {
      in.y = at(ws, w.oX2);
      in.y_stride_h = P; in.y_stride_l = H * P; in.y_stride_b = L * H * P;
    }
    if (a->final_state) in.final_state = reinterpret_cast<float*>(at(ws, w.oS1));
    int64_t clin = 0;
    const int rc = ssd_validate(&in, &clin);
    if (rc) return rc;
    if (w.copy_bc && L > 0) {
      e = mh::launch_col_copy(bc_in(a, a->B, a->B_stride_b, a->B_stride_l, at(ws, w.oB), w.ni, q), st);
      if (e == hipSuccess) e = mh::launch_col_copy(bc_in(a, a->C, a->C_stride_b, a->C_stride_l, at(ws, w.oC), w.ni, q), st);
    }
    if (e == hipSuccess && a->initial_state) e = mh::launch_col_copy(state_in(a, a->initial_state, at(ws, w.oS0), w.ni, q), st);
    if (e == hipSuccess) e = ssd_launch_native(&in, cl, ws, st);
    if (e == hipSuccess && a->final_state) e = mh::launch_col_copy(state_out(a, at(ws, w.oS1), a->final_state, w.ni, q), st);
  }
  if (e == hipSuccess && w.pieces == 2) {
    mh::RowAdd r{};
    r.es = es; r.d0 = b; r.d1 = L; r.d2 = H; r.ncols = P;
    r.dst = a->y; r.t0 = a->y_stride_b; r.t1 = a->y_stride_l; r.t2 = a->y_stride_h;
    r.src = at(ws, w.oX2); r.s2 = P; r.s1 = H * P; r.s0 = L * H * P;
    r.gate = a->z; r.g0 = a->z_stride_b; r.g1 = a->z_stride_l; r.g2 = a->z_stride_h;
    e = mh::launch_row_add(r, st);
  }
  return hip_status(e, "ssd_chunk_scan_fwd");
}

// Backward: oS0 = initial-state piece, oS1 = d_final_state piece, oH2 = d_initial_state piece; for two halves
// the second half's dx (oX2), ddt (oT2), dA and d_dt_bias (oH3) before they are added to the first half's.
void ssd_wide_bwd_plan(const mh_ssd_bwd_args* a, SsdWide& w) {
  const mh_ssd_args* f = &a->fwd;
  const int es = elem_size(f->dtype);
  const int64_t b = f->batch, L = f->seqlen, H = f->nheads, P = f->headdim, G = f->ngroups;
  w.ni = ssd_inner_dstate(f->dstate);
  w.pieces = f->dstate > 128 ? 2 : 1;
  w.copy_bc = f->dstate != w.pieces * w.ni || G > 1;
  w.inner = L > 0 ? mh::ssd_bwd_workspace_bytes((int)b, (int)L, (int)H, (int)w.ni, (int)G, f->dtype,
                                                ssd_bwd_heads_per_wg(f), (f->flags & MH_D_PER_CHANNEL) != 0) : 0;
  const size_t bc = w.copy_bc ? (size_t)(b * L * G * w.ni * es) : 0, st = (size_t)(b * H * P * w.ni * 4);
  size_t off = a256(w.inner);
  w.oB = off; off += a256(2 * bc);           // B piece, then dB piece
  w.oC = off; off += a256(2 * bc);           // C piece, then dC piece
  w.oS0 = off; off += f->initial_state ? a256(st) : 0;
  w.oS1 = off; off += a->d_final_state ? a256(st) : 0;
  w.oH2 = off; off += a->d_initial_state ? a256(st) : 0;
  const bool two = w.pieces == 2;
  w.oX2 = off; off += two ? a256((size_t)(b * L * H * P * es)) : 0;
  w.oT2 = off; off += two ? a256((size_t)(b * L * H * 4)) : 0;
  w.oH3 = off; off += two ? a256((size_t)(2 * H * 4)) : 0;
  w.total = off;
}

int ssd_bwd_wide(const mh_ssd_bwd_args* a, hipStream_t st) {
  const mh_ssd_args* f = &a->fwd;
  SsdWide w;
  ssd_wide_bwd_plan(a, w);
  void* ws = a->workspace;
  const int es = elem_size(f->dtype);
  const int64_t b = f->batch, L = f->seqlen, H = f->nheads, P = f->headdim, G = f->ngroups;
  const size_t bc = w.copy_bc ? (size_t)(b * L * G * w.ni * es) : 0;
  hipError_t e = hipSuccess;
  for (int q = 0; q < w.pieces && e == hipSuccess; ++q) {
    mh_ssd_bwd_args in = *a;
    in.fwd = ssd_piece(f, w, ws, q);
    in.fwd.workspace = nullptr; in.fwd.workspace_bytes = 0;
    in.d_final_state = a->d_final_state ? reinterpret_cast<const float*>(at(ws, w.oS1)) : nullptr;
    in.d_initial_state = a->d_initial_state ? reinterpret_cast<float*>(at(ws, w.oH2)) : nullptr;
    if (w.copy_bc) {
      in.dB = at(ws, w.oB + bc); in.dC = at(ws, w.oC + bc);
      in.dB_stride_l = in.dC_stride_l = G * w.ni;
      in.dB_stride_b = in.dC_stride_b = L * G * w.ni;
    } else {
      in.dB = at(a->dB, q * w.ni * es); in.dC = at(a->dC, q * w.ni * es);
    }
    if (q > 0) {
      in.dx = at(ws, w.oX2); in.dx_stride_h = P; in.dx_stride_l = H * P; in.dx_stride_b = L * H * P;
      in.dx_rows = nullptr;            // added once, by the first piece
      in.ddt = reinterpret_cast<float*>(at(ws, w.oT2)); in.ddt_stride_l = H; in.ddt_stride_b = L * H;
      in.dA = reinterpret_cast<float*>(at(ws, w.oH3));
      in.dD = nullptr;
      if (a->d_dt_bias) in.d_dt_bias = reinterpret_cast<float*>(at(ws, w.oH3)) + H;
    }
    in.workspace = ws; in.workspace_bytes = w.inner;
    const int rc = ssd_bwd_validate(&in);
    if (rc) return rc;
    if (w.copy_bc && L > 0) {
      e = mh::launch_col_copy(bc_in(f, f->B, f->B_stride_b, f->B_stride_l, at(ws, w.oB), w.ni, q), st);
      if (e == hipSuccess) e = mh::launch_col_copy(bc_in(f, f->C, f->C_stride_b, f->C_stride_l, at(ws, w.oC), w.ni, q), st);
    }
    if (e == hipSuccess && f->initial_state) e = mh::launch_col_copy(state_in(f, f->initial_state, at(ws, w.oS0), w.ni, q), st);
    if (e == hipSuccess && a->d_final_state) e = mh::launch_col_copy(state_in(f, a->d_final_state, at(ws, w.oS1), w.ni, q), st);
    if (e == hipSuccess) e = ssd_launch_bwd_native(&in, st);
    if (e == hipSuccess && w.copy_bc && L > 0) {
      e = mh::launch_col_copy(bc_out(f, at(ws, w.oB + bc), a->dB, a->dB_stride_b, a->dB_stride_l, w.ni, q), st);
      if (e == hipSuccess) e = mh::launch_col_copy(bc_out(f, at(ws, w.oC + bc), a->dC, a->dC_stride_b, a->dC_stride_l, w.ni, q), st);
    }
    if (e == hipSuccess && a->d_initial_state) e = mh::launch_col_copy(state_out(f, at(ws, w.oH2), a->d_initial_state, w.ni, q), st);
  }
  if (e == hipSuccess && w.pieces == 2) {
    mh::RowAdd r{};
    r.es = es; r.d0 = b; r.d1 = L; r.d2 = H; r.ncols = P;
    r.dst = a->dx; r.t0 = a->dx_stride_b; r.t1 = a->dx_stride_l; r.t2 = a->dx_stride_h;
    r.src = at(ws, w.oX2); r.s2 = P; r.s1 = H * P; r.s0 = L * H * P;
    e = mh::launch_row_add(r, st);
    if (e == hipSuccess) {
      mh::RowAdd t{};
      t.es = 4; t.d0 = b; t.d1 = L; t.d2 = 1; t.ncols = H;
      t.dst = a->ddt; t.t0 = a->ddt_stride_b; t.t1 = a->ddt_stride_l;
      t.src = at(ws, w.oT2); t.s0 = L * H; t.s1 = H;
      e = mh::launch_row_add(t, st);
    }
    for (int k = 0; k < 2 && e == hipSuccess; ++k) {
      float* dst = k == 0 ? a->dA : a->d_dt_bias;
      if (!dst) continue;
      mh::RowAdd t{};
      t.es = 4; t.d0 = t.d1 = t.d2 = 1; t.ncols = H;
      t.dst = dst; t.src = reinterpret_cast<float*>(at(ws, w.oH3)) + k * H;
      e = mh::launch_row_add(t, st);
    }
  }
  return hip_status(e, "ssd_chunk_scan_bwd");
}

// Workspace bytes of the forward (validated arguments, resolved chunk length) and of the backward.
size_t ssd_fwd_need(const mh_ssd_args* a, int64_t cl) {
  if (!ssd_native_dstate(a->dstate)) {
    SsdWide w;
    ssd_wide_fwd_plan(a, cl, w);
    return w.total;
  }
  const int64_t nchunks = (a->seqlen + cl - 1) / cl;
  return nchunks > 0 ? mh::ssd_workspace_bytes((int)a->batch, (int)a->seqlen, (int)nchunks, (int)a->nheads,
                                               (int)a->headdim, (int)a->dstate, (int)a->ngroups, a->dtype) : 0;
}
size_t ssd_bwd_need(const mh_ssd_bwd_args* a) {
  const mh_ssd_args* f = &a->fwd;
  if (!ssd_native_dstate(f->dstate)) {
    SsdWide w;
    ssd_wide_bwd_plan(a, w);
    return w.total;
  }
  return f->seqlen > 0 ? mh::ssd_bwd_workspace_bytes((int)f->batch, (int)f->seqlen, (int)f->nheads, (int)f->dstate,
                                                     (int)f->ngroups, f->dtype, ssd_bwd_heads_per_wg(f),
                                                     (f->flags & MH_D_PER_CHANNEL) != 0) : 0;
}

int conv_bwd_validate(const mh_conv1d_bwd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "conv1d_bwd: args is NULL");
  mh_conv1d_args f = a->fwd;
  f.y = const_cast<void*>(f.x);   // the forward output is not an input of the backward
  f.y_stride_b = f.x_stride_b;
  f.y_stride_l = f.x_stride_l;
  int rc = conv_validate(&f);
  if (rc) return rc;
  const int es = elem_size(f.dtype);
  if (!a->dweight) return fail(MH_ERR_NULL, "conv1d_bwd: dweight is required");
  if (f.bias && !a->dbias) return fail(MH_ERR_NULL, "conv1d_bwd: dbias is required when bias is given");
  if (f.seqlen > 0) {
    if (!a->dy || !a->dx) return fail(MH_ERR_NULL, "conv1d_bwd: dy and dx are required");
    if (!aligned16(a->dy) || !aligned16(a->dx)) return fail(MH_ERR_ALIGN, "conv1d_bwd: dy, dx must be 16-byte aligned");
    if (!stride_ok(a->dy_stride_b, es) || !stride_ok(a->dy_stride_l, es) || !stride_ok(a->dx_stride_b, es) ||
        !stride_ok(a->dx_stride_l, es))
      return fail(MH_ERR_ALIGN, "conv1d_bwd: strides must be multiples of 16 bytes");
    if (a->dy_stride_l < f.dim || a->dx_stride_l < f.dim)
      return fail(MH_ERR_STRIDE, "conv1d_bwd: token stride smaller than dim (channels must be contiguous)");
  }
  if (a->d_conv_state && f.conv_state_len > 0) {
    if (!aligned16(a->d_conv_state)) return fail(MH_ERR_ALIGN, "conv1d_bwd: d_conv_state must be 16-byte aligned");
    if (!stride_ok(a->d_conv_state_stride_b, es) || !stride_ok(a->d_conv_state_stride_l, es))
      return fail(MH_ERR_ALIGN, "conv1d_bwd: strides must be multiples of 16 bytes");
    if (a->d_conv_state_stride_l < f.dim)
      return fail(MH_ERR_STRIDE, "conv1d_bwd: token stride smaller than dim (channels must be contiguous)");
  }
  return MH_OK;
}

void conv_fill(const mh_conv1d_args* a, mh::Conv1dParams& p) {
  memset(&p, 0, sizeof(p));
  p.batch = (int)a->batch; p.seqlen = (int)a->seqlen; p.dim = (int)a->dim; p.width = (int)a->width;
  p.dtype = a->dtype; p.silu = (a->flags & MH_CONV_SILU) != 0;
  p.cs_len = (int)a->conv_state_len;
  p.x = a->x; p.x_sb = a->x_stride_b; p.x_sl = a->x_stride_l;
  p.weight = a->weight; p.bias = a->bias;
  p.conv_state = a->conv_state_len > 0 ? a->conv_state : nullptr;
  p.cs_sb = a->conv_state_stride_b; p.cs_sl = a->conv_state_stride_l;
  p.y = a->y; p.y_sb = a->y_stride_b; p.y_sl = a->y_stride_l;
}

void kda_fill(const mh_kda_args* a, mh::KdaParams& p) {
  memset(&p, 0, sizeof(p));
  p.batch = (int)a->batch; p.nheads = (int)a->nheads; p.seqlen = (int)a->seqlen; p.dk = (int)a->dk;
  p.dv = (int)a->dv; p.dtype = a->dtype; p.mode = a->mode;
  p.kernel_dim = a->kernel_dim < (int32_t)a->dk ? a->kernel_dim : (int32_t)a->dk;
  p.lam = a->lam; p.lam_h = a->lam_per_head;
  p.q1 = a->q1; p.q2 = a->q2; p.k = a->k; p.v = a->v; p.g = a->g;
  p.init_state = a->initial_state; p.init_z = a->initial_z;
  p.final_state = a->final_state; p.final_z = a->final_z;
  p.o = a->o; p.o2 = a->o2;
}

int kda_bwd_validate(const mh_kda_bwd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "kda_bwd: args is NULL");
  mh_kda_args f = a->fwd;
  if (!f.o) f.o = const_cast<void*>(f.v);   // the forward outputs are not inputs of the backward
  f.o2 = nullptr;
  int rc = kda_validate(&f);
  if (rc) return rc;
  if (f.mode != MH_KDA_REFERENCE)
    return fail(MH_ERR_UNSUPPORTED, "kda_bwd: only the reference mode has a backward (the gated operator has no "
                                    "reference training path)");
  if (a->flags & ~MH_KDA_BWD_DIFF) return fail(MH_ERR_UNSUPPORTED, "kda_bwd: unknown flags 0x%x", a->flags);
  const bool diff = (a->flags & MH_KDA_BWD_DIFF) != 0;
  if (diff && !f.q2 && f.seqlen > 0) return fail(MH_ERR_NULL, "kda_bwd: the differential output needs q2");
  if (diff && a->do2) return fail(MH_ERR_SHAPE, "kda_bwd: do2 is not used with the differential output");
  if (f.seqlen > 0 && !a->do1) return fail(MH_ERR_NULL, "kda_bwd: do1 is required");
  if (f.seqlen > 0 && (!a->dq1 || !a->dk || !a->dv || (f.q2 && !a->dq2)))
    return fail(MH_ERR_NULL, "kda_bwd: dq1, dk, dv (and dq2 with q2) are required");
  if (!f.q2 && f.seqlen > 0 && (a->dq2 || a->do2)) return fail(MH_ERR_NULL, "kda_bwd: dq2 / do2 given without q2");
  if (!aligned16(a->do1) || (a->do2 && !aligned16(a->do2)) || !aligned16(a->dq1) || (a->dq2 && !aligned16(a->dq2)) ||
      !aligned16(a->dk) || !aligned16(a->dv))
    return fail(MH_ERR_ALIGN, "kda_bwd: tensors must be 16-byte aligned");
  return MH_OK;
}

}  // namespace

extern "C" {

int mh_abi_version(void) { return MH_ABI_VERSION; }
const char* mh_last_error(void) { return g_err; }

int mh_ssd_chunk_len(const mh_ssd_args* a, int64_t* chunk_len) {
  if (!chunk_len) return fail(MH_ERR_NULL, "ssd: chunk_len output is NULL");
  return ssd_validate(a, chunk_len);
}

int mh_ssd_workspace_bytes(const mh_ssd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd: bytes output is NULL");
  int64_t cl = 0;
  int rc = ssd_validate(a, &cl);
  if (rc) return rc;
  *bytes = ssd_fwd_need(a, cl);
  return MH_OK;
}

int mh_ssd_chunk_scan_fwd(const mh_ssd_args* a, void* stream) {
  int64_t cl = 0;
  int rc = ssd_validate(a, &cl);
  if (rc) return rc;
  const size_t need = ssd_fwd_need(a, cl);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "ssd: workspace of %zu bytes (16-byte aligned) required, got %zu", need, a->workspace_bytes);
  if (!ssd_native_dstate(a->dstate)) return ssd_fwd_wide(a, cl, reinterpret_cast<hipStream_t>(stream));
  return hip_status(ssd_launch_native(a, cl, a->workspace, reinterpret_cast<hipStream_t>(stream)), "ssd_chunk_scan_fwd");
}

int mh_ssd_chunk_scan_fwd_noalloc(const mh_ssd_args* a, void* stream) {
  int64_t cl = 0;
  int rc = ssd_validate(a, &cl);
  if (rc) return rc;
  if (!ssd_native_dstate(a->dstate))
    return fail(MH_ERR_UNSUPPORTED, "ssd_noalloc: dstate %lld runs as a composition of 64/128-column scans that needs "
                "a caller workspace (call mh_ssd_chunk_scan_fwd)", (long long)a->dstate);
  const int64_t nchunks = (a->seqlen + cl - 1) / cl;
  const size_t need = mh::ssd_workspace_bytes((int)a->batch, (int)a->seqlen, (int)nchunks, (int)a->nheads,
                                              (int)a->headdim, (int)a->dstate, (int)a->ngroups, a->dtype);
  if (need > MH_NOALLOC_SCRATCH_BYTES)
    return fail(MH_ERR_WORKSPACE, "ssd_noalloc: these sizes need %zu bytes of workspace, more than the %zu-byte static "
                "scratch (call mh_ssd_chunk_scan_fwd with a caller workspace)", need, (size_t)MH_NOALLOC_SCRATCH_BYTES);
  mh::SsdParams p;
  ssd_fill(a, cl, nchunks, p);
  if (nchunks > 0) {
    void* ws = nullptr;
    rc = scratch_address(reinterpret_cast<hipStream_t>(stream), &ws);
    if (rc) return rc;
    mh::ssd_workspace_layout(p, ws);
  }
  return hip_status(mh::launch_ssd(p, reinterpret_cast<hipStream_t>(stream)), "ssd_chunk_scan_fwd_noalloc");
}

// h_states: the forward's argument block (y, final_state, z, chunk_len and the no-allocation scratch unused).
static int hs_validate(const mh_ssd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "ssd_h_states: args is NULL");
  mh_ssd_args g = *a;
  g.y = const_cast<void*>(g.x); g.y_stride_b = g.x_stride_b; g.y_stride_l = g.x_stride_l; g.y_stride_h = g.x_stride_h;
  g.z = nullptr;
  g.chunk_len = 64;
  int rc = ssd_validate(&g, nullptr);
  if (rc) return rc;
  if (!mh::ssd_hs_supported((int)a->nheads, (int)a->dstate))
    return fail(MH_ERR_UNSUPPORTED, "ssd_h_states: nheads %lld > 128 not supported", (long long)a->nheads);
  return MH_OK;
}

int mh_ssd_h_states_workspace_bytes(const mh_ssd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd_h_states: bytes output is NULL");
  int rc = hs_validate(a);
  if (rc) return rc;
  *bytes = mh::ssd_hs_workspace_bytes((int)a->batch, (int)a->seqlen, (int)a->nheads, (int)a->dstate,
                                      (int)a->ngroups, false);
  return MH_OK;
}

int mh_ssd_h_states(const mh_ssd_args* a, void* h_states, void* stream) {
  int rc = hs_validate(a);
  if (rc) return rc;
  if (a->seqlen > 0 && !h_states) return fail(MH_ERR_NULL, "ssd_h_states: h_states output is NULL");
  if (!aligned16(h_states)) return fail(MH_ERR_ALIGN, "ssd_h_states: h_states must be 16-byte aligned");
  const size_t need = mh::ssd_hs_workspace_bytes((int)a->batch, (int)a->seqlen, (int)a->nheads, (int)a->dstate,
                                                 (int)a->ngroups, false);
  if (a->seqlen > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "ssd_h_states: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  mh::SsdParams p;
  ssd_fill(a, 64, (a->seqlen + 63) / 64, p);
  mh::HsParams q;
  q.hs = h_states;
  if (a->seqlen > 0) mh::ssd_hs_workspace_layout(p, q, a->workspace, false);
  return hip_status(mh::launch_ssd_hs(p, q, reinterpret_cast<hipStream_t>(stream)), "ssd_h_states");
}

// ---------------------------------------------------------------- the reference's own scan form
static int rf_validate(const mh_ssd_args* a, bool h_states) {
  if (!a) return fail(MH_ERR_NULL, "ssd_ref_scan: args is NULL");
  if (a->batch <= 0 || a->seqlen < 0 || a->nheads <= 0 || a->headdim <= 0)
    return fail(MH_ERR_SHAPE, "ssd_ref_scan: batch, nheads, headdim must be positive and seqlen >= 0");
  const int64_t di = a->nheads * a->headdim;
  if (a->batch * di > 0x7fffffffLL || a->seqlen > 0x7fffffffLL / 16)
    return fail(MH_ERR_SHAPE, "ssd_ref_scan: sizes out of range");
  const int es = elem_size(a->dtype);
  if (!es) return fail(MH_ERR_DTYPE, "ssd_ref_scan: unknown dtype %d", a->dtype);
  if ((a->flags & (MH_A_PER_STATE | MH_DT_PER_CHANNEL)) != (MH_A_PER_STATE | MH_DT_PER_CHANNEL))
    return fail(MH_ERR_SHAPE, "ssd_ref_scan: the reference form takes MH_A_PER_STATE | MH_DT_PER_CHANNEL");
  if (!mh::ssd_rf_supported((int)a->dstate))
    return fail(MH_ERR_UNSUPPORTED, "ssd_ref_scan: dstate %lld not supported (16, 32, 64, 128, 256)",
                (long long)a->dstate);
  if (a->ngroups != 1) return fail(MH_ERR_UNSUPPORTED, "ssd_ref_scan: one group of B / C (ngroups 1)");
  if (di % 16) return fail(MH_ERR_UNSUPPORTED, "ssd_ref_scan: d_inner = nheads * headdim must be a multiple of 16");
  if ((a->flags & MH_DT_LIMIT) && !(a->dt_min <= a->dt_max)) return fail(MH_ERR_SHAPE, "ssd_ref_scan: dt_min > dt_max");
  if (!a->A) return fail(MH_ERR_NULL, "ssd_ref_scan: A is required");
  if (a->seqlen > 0 && (!a->x || !a->dt || !a->B || !a->C || !a->y))
    return fail(MH_ERR_NULL, "ssd_ref_scan: x, dt, A, B, C, y are required");
  if (a->x_stride_h != a->headdim || a->y_stride_h != a->headdim || (a->z && a->z_stride_h != a->headdim))
    return fail(MH_ERR_STRIDE, "ssd_ref_scan: the channels of a token (heads x headdim) must be contiguous in x, y, z");
  if (a->x_stride_l < di || a->y_stride_l < di || a->dt_stride_l < di || (a->z && a->z_stride_l < di))
    return fail(MH_ERR_STRIDE, "ssd_ref_scan: token stride smaller than d_inner");
  if (a->x_stride_b < 0 || a->dt_stride_b < 0 || a->y_stride_b < 0 || a->B_stride_b < 0 || a->C_stride_b < 0)
    return fail(MH_ERR_STRIDE, "ssd_ref_scan: negative batch stride");
  if (a->B_stride_l < a->dstate || a->C_stride_l < a->dstate)
    return fail(MH_ERR_STRIDE, "ssd_ref_scan: B / C token stride smaller than dstate");
  if (!aligned16(a->dt) || (a->dt_stride_l % 4) || (a->dt_stride_b % 4) || !aligned16(a->dt_bias))
    return fail(MH_ERR_ALIGN, "ssd_ref_scan: dt rows and dt_bias must be 16-byte aligned");
  if (!aligned16(a->B) || !aligned16(a->C) || !stride_ok(a->B_stride_b, es) || !stride_ok(a->B_stride_l, es) ||
      !stride_ok(a->C_stride_b, es) || !stride_ok(a->C_stride_l, es))
    return fail(MH_ERR_ALIGN, "ssd_ref_scan: B, C and their strides must be 16-byte aligned");
  if (!aligned16(a->y) || !stride_ok(a->y_stride_b, es) || !stride_ok(a->y_stride_l, es))
    return fail(MH_ERR_ALIGN, "ssd_ref_scan: y and its strides must be 16-byte aligned");
  (void)h_states;
  return MH_OK;
}

static void rf_fill(const mh_ssd_args* a, mh::RfParams& p) {
  p = mh::RfParams{};
  p.batch = (int)a->batch; p.seqlen = (int)a->seqlen; p.d_inner = (int)(a->nheads * a->headdim);
  p.headdim = (int)a->headdim; p.dstate = (int)a->dstate; p.dtype = a->dtype == MH_BF16 ? mh::DT_BF16 : mh::DT_F32;
  p.dt_softplus = (a->flags & MH_DT_SOFTPLUS) != 0;
  p.has_dt_limit = (a->flags & MH_DT_LIMIT) != 0;
  p.D_per_channel = (a->flags & MH_D_PER_CHANNEL) != 0;
  p.dt_min = a->dt_min; p.dt_max = a->dt_max;
  p.x = a->x; p.x_sb = a->x_stride_b; p.x_sl = a->x_stride_l;
  p.dt = a->dt; p.dt_sb = a->dt_stride_b; p.dt_sl = a->dt_stride_l;
  p.A = a->A;
  p.B = a->B; p.B_sb = a->B_stride_b; p.B_sl = a->B_stride_l;
  p.C = a->C; p.C_sb = a->C_stride_b; p.C_sl = a->C_stride_l;
  p.D = a->D; p.dt_bias = a->dt_bias; p.init_state = a->initial_state;
  p.y = a->y; p.y_sb = a->y_stride_b; p.y_sl = a->y_stride_l;
  p.z = a->z; p.z_sb = a->z_stride_b; p.z_sl = a->z_stride_l;
  p.final_state = a->final_state;
}

static int hs_bwd_validate(const mh_ssd_hs_bwd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "ssd_h_states_bwd: args is NULL");
  int rc = hs_validate(&a->fwd);
  if (rc) return rc;
  const mh_ssd_args* f = &a->fwd;
  if (!mh::ssd_hs_bwd_supported((int)f->nheads, (int)f->dstate))
    return fail(MH_ERR_UNSUPPORTED, "ssd_h_states_bwd: nheads %lld / dstate %lld not supported (<= 128 each)",
                (long long)f->nheads, (long long)f->dstate);
  if (!a->dA) return fail(MH_ERR_NULL, "ssd_h_states_bwd: dA is NULL");
  if (f->dt_bias && !a->d_dt_bias) return fail(MH_ERR_NULL, "ssd_h_states_bwd: d_dt_bias is NULL while dt_bias is set");
  if (f->seqlen > 0 && (!a->dhs || !(a->dx || a->dx_rows) || !a->ddt || !a->dB))
    return fail(MH_ERR_NULL, "ssd_h_states_bwd: dhs, dx (or dx_rows), ddt and dB are required");
  if (!aligned16(a->dhs) || !aligned16(a->dx) || !aligned16(a->dB) || !aligned16(a->d_initial_state))
    return fail(MH_ERR_ALIGN, "ssd_h_states_bwd: dhs, dx, dB and d_initial_state must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(a->dx_rows) % 4)
    return fail(MH_ERR_ALIGN, "ssd_h_states_bwd: dx_rows must be 4-byte aligned");
  return MH_OK;
}

// ---------------------------------------------------------------- output gate (training path)
static int gate_validate(const mh_gate_args* a, bool bwd) {
  if (!a) return fail(MH_ERR_NULL, "silu_gate: args is NULL");
  if (a->batch < 0 || a->seqlen < 0 || a->nheads < 0 || a->headdim <= 0)
    return fail(MH_ERR_SHAPE, "silu_gate: sizes must be non-negative (headdim positive)");
  if (a->headdim % 8) return fail(MH_ERR_UNSUPPORTED, "silu_gate: headdim must be a multiple of 8");
  const int es = elem_size(a->dtype);
  if (!es) return fail(MH_ERR_DTYPE, "silu_gate: unknown dtype %d", a->dtype);
  if (a->batch * a->seqlen * a->nheads == 0) return MH_OK;
  if (!a->y || !a->z || !a->out || (bwd && (!a->g || !a->dz)))
    return fail(MH_ERR_NULL, bwd ? "silu_gate_bwd: y, z, g, out (dy), dz are required"
                                 : "silu_gate_fwd: y, z, out are required");
  const void* ptrs[5] = {a->y, a->z, a->out, bwd ? a->g : a->y, bwd ? a->dz : a->y};
  const int64_t strides[5][3] = {{a->y_stride_b, a->y_stride_l, a->y_stride_h},
                                 {a->z_stride_b, a->z_stride_l, a->z_stride_h},
                                 {a->out_stride_b, a->out_stride_l, a->out_stride_h},
                                 {a->g_stride_b, a->g_stride_l, a->g_stride_h},
                                 {a->dz_stride_b, a->dz_stride_l, a->dz_stride_h}};
  for (int i = 0; i < (bwd ? 5 : 3); ++i) {
    if (!aligned16(ptrs[i])) return fail(MH_ERR_ALIGN, "silu_gate: tensors must be 16-byte aligned");
    for (int k = 0; k < 3; ++k)
      if (strides[i][k] < 0 || !stride_ok(strides[i][k], es))
        return fail(MH_ERR_ALIGN, "silu_gate: strides must be non-negative multiples of 16 bytes");
  }
  return MH_OK;
}

static hipError_t gate_launch(const mh_gate_args* a, bool bwd, hipStream_t st) {
  mh::GateParams g{};
  g.es = elem_size(a->dtype);
  g.d0 = a->batch; g.d1 = a->seqlen; g.d2 = a->nheads; g.ncols = a->headdim;
  g.y = a->y; g.y0 = a->y_stride_b; g.y1 = a->y_stride_l; g.y2 = a->y_stride_h;
  g.z = a->z; g.z0 = a->z_stride_b; g.z1 = a->z_stride_l; g.z2 = a->z_stride_h;
  g.g = a->g; g.g0 = a->g_stride_b; g.g1 = a->g_stride_l; g.g2 = a->g_stride_h;
  g.out = a->out; g.o0 = a->out_stride_b; g.o1 = a->out_stride_l; g.o2 = a->out_stride_h;
  g.dz = a->dz; g.dz0 = a->dz_stride_b; g.dz1 = a->dz_stride_l; g.dz2 = a->dz_stride_h;
  return mh::launch_gate(g, bwd, st);
}

int mh_silu_gate_fwd(const mh_gate_args* a, void* stream) {
  const int rc = gate_validate(a, false);
  if (rc) return rc;
  return hip_status(gate_launch(a, false, reinterpret_cast<hipStream_t>(stream)), "silu_gate_fwd");
}

int mh_silu_gate_bwd(const mh_gate_args* a, void* stream) {
  const int rc = gate_validate(a, true);
  if (rc) return rc;
  return hip_status(gate_launch(a, true, reinterpret_cast<hipStream_t>(stream)), "silu_gate_bwd");
}

int mh_ssd_ref_scan_workspace_bytes(const mh_ssd_args* a, int h_states, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd_ref_scan: bytes output is NULL");
  const int rc = rf_validate(a, h_states != 0);
  if (rc) return rc;
  *bytes = mh::ssd_rf_workspace_bytes((int)a->batch, (int)a->seqlen, (int)(a->nheads * a->headdim), (int)a->dstate,
                                      h_states != 0);
  return MH_OK;
}

int mh_ssd_ref_scan_fwd(const mh_ssd_args* a, void* h_states, void* stream) {
  const int rc = rf_validate(a, h_states != nullptr);
  if (rc) return rc;
  const size_t need = mh::ssd_rf_workspace_bytes((int)a->batch, (int)a->seqlen, (int)(a->nheads * a->headdim),
                                                 (int)a->dstate, h_states != nullptr);
  if (need && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "ssd_ref_scan: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  mh::RfParams p;
  rf_fill(a, p);
  p.hs = h_states;
  p.hs_part = reinterpret_cast<float*>(a->workspace);
  return hip_status(mh::launch_ssd_rf(p, reinterpret_cast<hipStream_t>(stream)), "ssd_ref_scan");
}

static int rf_bwd_validate(const mh_ssd_ref_bwd_args* a) {
  if (!a) return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: args is NULL");
  // the forward's checks, with the output the backward does not write taken from x
  mh_ssd_args g = a->fwd;
  if (g.z) return fail(MH_ERR_UNSUPPORTED, "ssd_ref_scan_bwd: the output gate is not differentiated here (fwd.z must be NULL)");
  g.y = const_cast<void*>(g.x); g.y_stride_b = g.x_stride_b; g.y_stride_l = g.x_stride_l; g.y_stride_h = g.x_stride_h;
  int rc = rf_validate(&g, false);
  if (rc) return rc;
  const mh_ssd_args* f = &a->fwd;
  if (f->seqlen > 0 && (!a->dx || !a->ddt || !a->dB || !a->dC))
    return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: dx, ddt, dB and dC are required");
  if (!a->dA) return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: dA is required");
  if (f->D && !a->dD) return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: dD is required when D is given");
  if (f->dt_bias && !a->d_dt_bias) return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: d_dt_bias is required with dt_bias");
  const int es = elem_size(f->dtype);
  const uintptr_t m = (uintptr_t)es - 1;
  if (((uintptr_t)a->dy & m) || ((uintptr_t)a->dhs & m) || ((uintptr_t)a->dx & m) || ((uintptr_t)a->dB & m) ||
      ((uintptr_t)a->dC & m) || ((uintptr_t)a->ddt & 3) || ((uintptr_t)a->d_final_state & 3) ||
      ((uintptr_t)a->d_initial_state & 3))
    return fail(MH_ERR_ALIGN, "ssd_ref_scan_bwd: gradient pointers must be aligned to their element size");
  return MH_OK;
}

static size_t rf_bwd_need(const mh_ssd_ref_bwd_args* a) {
  const mh_ssd_args* f = &a->fwd;
  return mh::ssd_rf_bwd_workspace_bytes((int)f->batch, (int)f->seqlen, (int)(f->nheads * f->headdim), (int)f->dstate);
}

int mh_ssd_ref_scan_bwd_workspace_bytes(const mh_ssd_ref_bwd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd_ref_scan_bwd: bytes output is NULL");
  const int rc = rf_bwd_validate(a);
  if (rc) return rc;
  *bytes = rf_bwd_need(a);
  return MH_OK;
}

int mh_ssd_ref_scan_bwd(const mh_ssd_ref_bwd_args* a, void* stream) {
  const int rc = rf_bwd_validate(a);
  if (rc) return rc;
  const size_t need = rf_bwd_need(a);
  if (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace))
    return fail(MH_ERR_WORKSPACE, "ssd_ref_scan_bwd: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  mh::RfParams p;
  rf_fill(&a->fwd, p);
  p.y = nullptr;
  p.z = nullptr;
  p.final_state = nullptr;
  p.dy = a->dy; p.dhs = a->dhs; p.d_final = a->d_final_state;
  p.dx = a->dx; p.ddt = a->ddt; p.dA = a->dA; p.dB = a->dB; p.dC = a->dC;
  p.dD = a->fwd.D ? a->dD : nullptr;
  p.d_dt_bias = a->fwd.dt_bias ? a->d_dt_bias : nullptr;
  p.dh0 = a->d_initial_state;
  mh::ssd_rf_bwd_layout(p, a->workspace);
  return hip_status(mh::launch_ssd_rf_bwd(p, reinterpret_cast<hipStream_t>(stream)), "ssd_ref_scan_bwd");
}

int mh_ssd_h_states_bwd_workspace_bytes(const mh_ssd_hs_bwd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd_h_states_bwd: bytes output is NULL");
  int rc = hs_bwd_validate(a);
  if (rc) return rc;
  const mh_ssd_args* f = &a->fwd;
  *bytes = mh::ssd_hs_workspace_bytes((int)f->batch, (int)f->seqlen, (int)f->nheads, (int)f->dstate,
                                      (int)f->ngroups, true);
  return MH_OK;
}

int mh_ssd_h_states_bwd(const mh_ssd_hs_bwd_args* a, void* stream) {
  int rc = hs_bwd_validate(a);
  if (rc) return rc;
  const mh_ssd_args* f = &a->fwd;
  const size_t need = mh::ssd_hs_workspace_bytes((int)f->batch, (int)f->seqlen, (int)f->nheads, (int)f->dstate,
                                                 (int)f->ngroups, true);
  if (f->seqlen > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "ssd_h_states_bwd: workspace of %zu bytes (16-byte aligned) required, got %zu",
                need, a->workspace_bytes);
  mh::SsdParams p;
  ssd_fill(f, 64, (f->seqlen + 63) / 64, p);
  mh::HsParams q;
  memset(&q, 0, sizeof(q));
  q.dhs = a->dhs; q.dx = a->dx; q.ddt = a->ddt; q.dA = a->dA; q.dB = a->dB; q.dx_rows = a->dx_rows;
  q.d_dt_bias = f->dt_bias ? a->d_dt_bias : nullptr;
  if (f->seqlen > 0) mh::ssd_hs_workspace_layout(p, q, a->workspace, true);
  else p.nseg = 0;
  return hip_status(mh::launch_ssd_hs_bwd(p, q, a->d_initial_state, reinterpret_cast<hipStream_t>(stream)),
                    "ssd_h_states_bwd");
}

int mh_ssd_state_update(const mh_ssu_args* a, void* stream) {
  int rc = ssu_validate(a);
  if (rc) return rc;
  mh::SsuParams p;
  memset(&p, 0, sizeof(p));
  p.batch = (int)a->batch; p.nheads = (int)a->nheads; p.headdim = (int)a->headdim; p.dstate = (int)a->dstate;
  p.ngroups = (int)a->ngroups; p.dtype = a->dtype;
  p.dt_softplus = (a->flags & MH_DT_SOFTPLUS) != 0;
  p.has_dt_limit = (a->flags & MH_DT_LIMIT) != 0;
  p.D_per_channel = (a->flags & MH_D_PER_CHANNEL) != 0;
  p.A_per_state = (a->flags & MH_A_PER_STATE) != 0;
  p.dt_per_channel = (a->flags & MH_DT_PER_CHANNEL) != 0;
  p.dt_min = a->dt_min; p.dt_max = a->dt_max;
  p.state_in = a->state_in; p.state_out = a->state_out;
  p.x = a->x; p.x_stride_b = a->x_stride_b;
  p.dt = a->dt; p.dt_stride_b = a->dt_stride_b;
  p.A = a->A;
  p.B = a->B; p.B_stride_b = a->B_stride_b;
  p.C = a->C; p.C_stride_b = a->C_stride_b;
  p.D = a->D; p.dt_bias = a->dt_bias;
  p.y = a->y; p.y_stride_b = a->y_stride_b;
  p.z = a->z; p.z_stride_b = a->z_stride_b;
  return hip_status(mh::launch_ssu(p, reinterpret_cast<hipStream_t>(stream)), "ssd_state_update");
}

int mh_kda_chunk_scan_fwd(const mh_kda_args* a, void* stream) {
  int rc = kda_validate(a);
  if (rc) return rc;
  mh::KdaParams p;
  kda_fill(a, p);
  return hip_status(mh::launch_kda(p, reinterpret_cast<hipStream_t>(stream)), "kda_chunk_scan_fwd");
}

int mh_kda_bwd_workspace_bytes(const mh_kda_bwd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "kda_bwd: bytes output is NULL");
  int rc = kda_bwd_validate(a);
  if (rc) return rc;
  const mh_kda_args* f = &a->fwd;
  *bytes = mh::kda_bwd_workspace_bytes((int)f->batch, (int)f->nheads, (int)f->seqlen, f->q2 ? 2 : 1);
  return MH_OK;
}

int mh_kda_chunk_scan_bwd(const mh_kda_bwd_args* a, void* stream) {
  int rc = kda_bwd_validate(a);
  if (rc) return rc;
  const mh_kda_args* f = &a->fwd;
  const int nq = f->q2 ? 2 : 1;
  const size_t need = mh::kda_bwd_workspace_bytes((int)f->batch, (int)f->nheads, (int)f->seqlen, nq);
  if (f->seqlen > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "kda_bwd: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  mh::KdaBwdParams q;
  memset(&q, 0, sizeof(q));
  kda_fill(f, q.f);
  q.f.o = nullptr; q.f.o2 = nullptr; q.f.final_state = nullptr; q.f.final_z = nullptr;
  q.nq = nq;
  q.diff = (a->flags & MH_KDA_BWD_DIFF) != 0;
  q.do1 = a->do1; q.do2 = q.diff ? nullptr : a->do2;
  q.d_final = a->d_final_state; q.d_final_z = a->d_final_z;
  q.dq1 = a->dq1; q.dq2 = a->dq2; q.dk = a->dk; q.dv = a->dv;
  q.dS0 = a->d_initial_state; q.dz0 = a->d_initial_z;
  q.dlam = q.diff ? a->d_lam : nullptr;
  if (f->seqlen > 0) mh::kda_bwd_workspace_layout(q, a->workspace);
  return hip_status(mh::launch_kda_bwd(q, reinterpret_cast<hipStream_t>(stream)), "kda_chunk_scan_bwd");
}

int mh_kda_recurrent_step(const mh_kda_step_args* a, void* stream) {
  int rc = kda_step_validate(a);
  if (rc) return rc;
  mh::KdaStepParams p;
  memset(&p, 0, sizeof(p));
  p.batch = (int)a->batch; p.nheads = (int)a->nheads; p.dk = (int)a->dk; p.dv = (int)a->dv; p.dtype = a->dtype;
  p.apply_phi = (a->flags & MH_KDA_PHI) != 0;
  p.kernel_dim = p.apply_phi ? (a->kernel_dim < (int32_t)a->dk ? a->kernel_dim : (int32_t)a->dk) : (int)a->dk;
  p.lam = a->lam; p.lam_h = a->lam_per_head;
  p.q1 = a->q1; p.q2 = a->q2; p.k = a->k; p.v = a->v;
  p.state = a->state; p.z = a->z; p.o = a->o; p.o2 = a->o2;
  return hip_status(mh::launch_kda_step(p, reinterpret_cast<hipStream_t>(stream)), "kda_recurrent_step");
}

int mh_causal_conv1d_fwd(const mh_conv1d_args* a, void* stream) {
  int rc = conv_validate(a);
  if (rc) return rc;
  mh::Conv1dParams p;
  conv_fill(a, p);
  return hip_status(mh::launch_conv1d(p, reinterpret_cast<hipStream_t>(stream)), "causal_conv1d_fwd");
}

int mh_conv1d_bwd_workspace_bytes(const mh_conv1d_bwd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "conv1d_bwd: bytes output is NULL");
  int rc = conv_bwd_validate(a);
  if (rc) return rc;
  *bytes = mh::conv1d_bwd_workspace_bytes((int)a->fwd.batch, (int)a->fwd.seqlen, (int)a->fwd.dim, (int)a->fwd.width);
  return MH_OK;
}

int mh_causal_conv1d_bwd(const mh_conv1d_bwd_args* a, void* stream) {
  int rc = conv_bwd_validate(a);
  if (rc) return rc;
  const mh_conv1d_args* f = &a->fwd;
  const size_t need = mh::conv1d_bwd_workspace_bytes((int)f->batch, (int)f->seqlen, (int)f->dim, (int)f->width);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "conv1d_bwd: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  mh::Conv1dBwdParams q;
  memset(&q, 0, sizeof(q));
  conv_fill(f, q.f);
  q.f.y = nullptr;
  q.dy = a->dy; q.dy_sb = a->dy_stride_b; q.dy_sl = a->dy_stride_l;
  q.dx = a->dx; q.dx_sb = a->dx_stride_b; q.dx_sl = a->dx_stride_l;
  q.dweight = a->dweight; q.dbias = f->bias ? a->dbias : nullptr;
  if (f->conv_state_len > 0 && a->d_conv_state) {
    q.dcs = a->d_conv_state; q.dcs_sb = a->d_conv_state_stride_b; q.dcs_sl = a->d_conv_state_stride_l;
  }
  mh::conv1d_bwd_workspace_layout(q, a->workspace);
  return hip_status(mh::launch_conv1d_bwd(q, reinterpret_cast<hipStream_t>(stream)), "causal_conv1d_bwd");
}

int mh_ssd_bwd_workspace_bytes(const mh_ssd_bwd_args* a, size_t* bytes) {
  if (!bytes) return fail(MH_ERR_NULL, "ssd_bwd: bytes output is NULL");
  int rc = ssd_bwd_validate(a);
  if (rc) return rc;
  *bytes = ssd_bwd_need(a);
  return MH_OK;
}

int mh_ssd_chunk_scan_bwd(const mh_ssd_bwd_args* a, void* stream) {
  int rc = ssd_bwd_validate(a);
  if (rc) return rc;
  const mh_ssd_args* f = &a->fwd;
  const size_t need = ssd_bwd_need(a);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned16(a->workspace)))
    return fail(MH_ERR_WORKSPACE, "ssd_bwd: workspace of %zu bytes (16-byte aligned) required, got %zu", need,
                a->workspace_bytes);
  if (!ssd_native_dstate(f->dstate)) return ssd_bwd_wide(a, reinterpret_cast<hipStream_t>(stream));
  return hip_status(ssd_launch_bwd_native(a, reinterpret_cast<hipStream_t>(stream)), "ssd_chunk_scan_bwd");
}

}  // extern "C"
