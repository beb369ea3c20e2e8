"""mamformer_amd -- MI355X (gfx950) implementation of Mamformer's Mamba-2 SSD / KDA scan path.

Public ops (``mamformer_amd.ops``): ``selective_scan`` (SSD chunked-scan
prefill, differentiable) and ``selective_scan_bwd`` (its backward), ``selective_state_update`` / ``recurrent_step`` (decode step) and
``linear_attn_scan`` (KDA gated scan), ``causal_conv1d`` (Mamba layer
prologue); layer-level counterparts in ``mamformer_amd.layers``.  They run hand-written HIP kernels from
``libmamformer_hip.so`` (build with ``python -m mamformer_amd.build``).
"""

from .ops import (Plan, causal_conv1d, diff_lambda, linear_attention_recurrent, linear_attention_scan, linear_attn_scan,
                  linear_attn_scan_pair, linear_attn_scan_single, linear_attn_step, plan_linear_attn_scan,
                  plan_linear_attn_step, plan_selective_scan, plan_selective_scan_bwd, plan_selective_state_update, recurrent_step,
                  recurrent_step_reference, selective_scan_reference, plan_selective_scan_reference,
                  selective_scan, selective_scan_bwd, selective_state_update, ssd_chunk_len, linear_attn_scan_bwd)

__all__ = ["selective_scan", "selective_scan_bwd", "selective_state_update", "recurrent_step", "recurrent_step_reference", "selective_scan_reference",
           "plan_selective_scan_reference", "linear_attn_scan",
           "linear_attn_scan_pair", "linear_attn_scan_single", "linear_attention_scan", "diff_lambda",
           "linear_attn_step", "linear_attention_recurrent",
           "ssd_chunk_len", "Plan", "plan_selective_scan", "plan_selective_scan_bwd", "plan_selective_state_update", "plan_linear_attn_scan",
           "plan_linear_attn_step", "causal_conv1d", "linear_attn_scan_bwd", "layers"]

from . import layers  # noqa: E402  (layer-level counterparts: Mamba2Layer, kda_linear_attention)
