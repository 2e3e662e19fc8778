"""ConcordLinearPackedB on MI355X: the packed-weight linear layer whose optimizer
step runs inside its own backward.

Drop-in for concord/packed_b.py (reference, file:line cited per function).
Each weight is one int32 word -- s_fast int16 (bits 31..16), s_slow int8
(15..8), v_slow int8 (7..0) -- on shared per-row/per-column int8 exponents:

    W = (s_fast + 128 s_slow + 128 v_slow) * 2^(row_exp + col_exp - 15)

All compute runs in libconcord_amd.so (hand-written gfx950 kernels, C ABI in
include/concord_amd.h).  There is no CPU path: layers must live on a ROCm
device and every compute call raises if the library is missing.

Two forward/dgrad modes, both bit-identical in what they feed the MFMAs:
  weight_cache=False (default)  fused dequant-GEMM: packed words are decoded
                                into LDS tiles; no bf16 weight copy is kept.
  weight_cache=True             the reference's dataflow: the update emits a
                                bf16 weight_buf (materialize-merge) and the
                                GEMMs read it.
"""
import ctypes
import math

import torch
import torch.nn as nn

from . import _lib as C

MANTISSA_BIAS = 15
INT8_MIN, INT8_MAX = -128, 127
INT16_MIN, INT16_MAX = -32768, 32767
S_SLOW_FACTOR = 128
V_SLOW_FACTOR = 128


def compute_drift_cancel_C(alpha, alpha_v_fast, alpha_v_slow=0.0, refit_period=1,
                           mass_preserve=True):
    """Drift-cancellation coefficient C* (concord/packed_b.py:52-102).

    L = (1-alpha)/alpha, rho = alpha_v_fast + alpha_v_slow/T_r.  Mass-preserving
    leak: C* = L*2rho/(1-2rho) (0.018036 at the defaults); legacy:
    C* = L*rho/(1 - L*alpha_v_fast) (0.00908)."""
    L = (1.0 - alpha) / max(alpha, 1e-12)
    rho = alpha_v_fast + alpha_v_slow / max(refit_period, 1)
    if mass_preserve:
        rho2 = 2.0 * rho
        return L * rho2 / (1.0 - rho2)
    return L * rho / (1.0 - L * alpha_v_fast)


# ---------------------------------------------------------------------------
# Module-global switches (concord/packed_b.py:797-860; prototype additions
# notebook/src/prototype_packed_b.py:325-353, 1016-1051)
# ---------------------------------------------------------------------------
_USE_FIXED_COH = True
_GATE_GAIN = 1.0
_COH_WEIGHTED_V = False
_RATIO_COH = False
# the v-hat finalize and the adamw update carried by the backward's WGRAD
# launch (concord_dgrad_wgrad_update) instead of launches of their own
_FUSED_UPDATE = False
_RATIO_CHASE_FLOOR = 0.9
_RATIO_LEAK_FLOOR = 0.999
_PROTO_SEMANTICS = False


def set_fixed_coh(enabled):
    global _USE_FIXED_COH
    _USE_FIXED_COH = bool(enabled)


def set_gate_gain(g):
    global _GATE_GAIN
    _GATE_GAIN = float(g)


def set_coh_weighted_v(enabled):
    """Experimental coh_pre-weighted v-hat accumulation (concord/packed_b.py:828-833).
    Not implemented on this path; enabling it raises."""
    global _COH_WEIGHTED_V
    if enabled:
        raise NotImplementedError(
            "concord_amd: the coh_pre-weighted v-hat (experimental, default off) is not implemented")
    _COH_WEIGHTED_V = False


def set_ratio_coh(enabled):
    global _RATIO_COH
    _RATIO_COH = bool(enabled)


def set_fused_update(enabled):
    """True: the fused-forward layer's backward with the v-hat drive runs the
    v-hat finalize and the adamw update inside its WGRAD launch when the
    update's flags allow it (concord_dgrad_wgrad_update with fuse); False
    (default): launches of their own.  The results are the same either way."""
    global _FUSED_UPDATE
    _FUSED_UPDATE = bool(enabled)


def set_ratio_coh_floors(chase, leak):
    """Per-step floors of the ratio-coherence gates.  The kernels read them from
    per-device fp32[1] tensors, so a captured graph sees the update
    (notebook/src/prototype_packed_b.py:1005-1013)."""
    global _RATIO_CHASE_FLOOR, _RATIO_LEAK_FLOOR
    _RATIO_CHASE_FLOOR = float(chase)
    _RATIO_LEAK_FLOOR = float(leak)
    for t in _CHASE_FLOOR_T.values():
        t.fill_(_RATIO_CHASE_FLOOR)
    for t in _LEAK_FLOOR_T.values():
        t.fill_(_RATIO_LEAK_FLOOR)


def set_prototype_semantics(enabled):
    """Switch the update between concord/packed_b.py:422-703 (False, default) and
    notebook/src/prototype_packed_b.py:454-778 (True): consolidate-gated
    chase/leak/decay/weight-emit/watermarks, coherence-gated beta1
    (+consf*beta1*coh*s_fast instead of -beta1*s_fast) and the v-hat
    bias-correction factor.  Identical at beta1 = 0, consolidate = 1, v_bc = 1."""
    global _PROTO_SEMANTICS
    _PROTO_SEMANTICS = bool(enabled)


# ---------------------------------------------------------------------------
# Per-device device scalars (concord/packed_b.py:315-359; prototype 331-353,
# 1016-1046)
# ---------------------------------------------------------------------------
def _dev_key(device):
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    return str(d)


_STEP_COUNTERS = {}
_LR_SCALAR_CACHE = {}
_EPS_SCALAR_CACHE = {}
_CHASE_FLOOR_T = {}
_LEAK_FLOOR_T = {}
_CONSOLIDATE_FLAGS = {}
_V_BC_BUFS = {}
_REB_SEED_CACHE = {}
_WORKSPACES = {}


def _get_step_counter(device):
    """The SR salt counter shared by every layer on a device, advanced once per
    update (concord/packed_b.py:315-322, 910-911)."""
    key = _dev_key(device)
    if key not in _STEP_COUNTERS:
        _STEP_COUNTERS[key] = torch.zeros(1, dtype=torch.int32, device=key)
    return _STEP_COUNTERS[key]


def _scalar_tensor(cache, value, device, dtype=torch.float32):
    if isinstance(value, torch.Tensor):
        return value
    key = _dev_key(device)
    buf = cache.get(key)
    if buf is None:
        buf = torch.zeros(1, dtype=dtype, device=key)
        cache[key] = buf
    buf.fill_(value)
    return buf


def _ensure_lr_tensor(lr, device):
    return _scalar_tensor(_LR_SCALAR_CACHE, float(lr) if not isinstance(lr, torch.Tensor) else lr, device)


def _ensure_eps_tensor(eps, device):
    return _scalar_tensor(_EPS_SCALAR_CACHE, float(eps) if not isinstance(eps, torch.Tensor) else eps, device)


def _ensure_floor_tensors(device):
    key = _dev_key(device)
    if key not in _CHASE_FLOOR_T:
        _CHASE_FLOOR_T[key] = torch.full((1,), _RATIO_CHASE_FLOOR, dtype=torch.float32, device=key)
        _LEAK_FLOOR_T[key] = torch.full((1,), _RATIO_LEAK_FLOOR, dtype=torch.float32, device=key)
    return _CHASE_FLOOR_T[key], _LEAK_FLOOR_T[key]


def _get_consolidate_flag(device):
    key = _dev_key(device)
    if key not in _CONSOLIDATE_FLAGS:
        _CONSOLIDATE_FLAGS[key] = torch.ones(1, dtype=torch.int32, device=key)
    return _CONSOLIDATE_FLAGS[key]


def set_consolidate(device, consolidate):
    """Gradient-accumulation gate (notebook/src/prototype_packed_b.py:348-353):
    False for the first micro-steps of a cycle (tick-only), True for the last.
    Turns on the prototype update semantics.  With weight_cache=False the
    forward decodes the live words, so use weight_cache=True to keep the
    forward weights frozen through a cycle as the prototype does."""
    set_prototype_semantics(True)
    _get_consolidate_flag(device).fill_(1 if consolidate else 0)


def _v_bc_buf(device):
    key = _dev_key(device)
    if key not in _V_BC_BUFS:
        _V_BC_BUFS[key] = torch.ones(1, dtype=torch.float32, device=key)
    return _V_BC_BUFS[key]


def set_v_bias_correction(factor):
    """Fill the per-device v-hat bias-correction factor 1/(1-beta2^t)
    (notebook/src/prototype_packed_b.py:1042-1046); turns on the prototype
    update semantics."""
    set_prototype_semantics(True)
    for buf in _V_BC_BUFS.values():
        buf.fill_(float(factor))


def bias_correction_factor(step, beta2=0.999):
    return 1.0 / (1.0 - beta2 ** (int(step) + 1))


def _ensure_reb_seed_tensor(device):
    key = _dev_key(device)
    if key not in _REB_SEED_CACHE:
        _REB_SEED_CACHE[key] = torch.zeros(1, dtype=torch.int32, device=key)
    return _REB_SEED_CACHE[key]


_GEMM_WORKSPACES = {}


def _gemm_workspace(device, M, N, K):
    """Zero-initialised per-device split-K workspace of the GEMMs, grown to the
    largest problem seen (grow it eagerly, before any graph capture)."""
    key = _dev_key(device)
    need = int(C.lib().concord_gemm_workspace_bytes(int(M), int(N), int(K)))
    ws = _GEMM_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=key)
        _GEMM_WORKSPACES[key] = ws
    return ws


def _workspace(device, N, K, M=0):
    """Zero-initialised per-device workspace, grown to the largest layer."""
    key = _dev_key(device)
    need = int(C.lib().concord_workspace_bytes(int(N), int(K), int(M)))
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=key)
        _WORKSPACES[key] = ws
    return ws


# ---------------------------------------------------------------------------
# Rebalance statistics (concord/packed_b.py:1098-1111)
# ---------------------------------------------------------------------------
_REB_STATS = None


def reset_reb_stats():
    global _REB_STATS
    _REB_STATS = dict(calls=0, tickup_dim=0, tickdown_dim=0, dim_total=0,
                      clip_elems=0, elem_total=0)


def get_reb_stats():
    return _REB_STATS


# ---------------------------------------------------------------------------
# Launch wrappers (same names and argument meaning as the reference)
# ---------------------------------------------------------------------------
def _check_packed(packed_w, row_exp, col_exp):
    C.require_device_tensor(packed_w, "packed_w")
    if packed_w.dtype != torch.int32 or packed_w.dim() != 2 or packed_w.stride(1) != 1:
        raise AssertionError("packed_w must be a row-major [N, K] int32 tensor")
    N, K = packed_w.shape
    if row_exp.dtype != torch.int8 or col_exp.dtype != torch.int8:
        raise AssertionError("row_exp / col_exp must be int8")
    if row_exp.numel() != N or col_exp.numel() != K:
        raise AssertionError("row_exp / col_exp sizes do not match packed_w")
    return N, K


def materialize_packed_bf16(packed_w, row_exp, col_exp, out, mantissa_bias=15,
                            consolidated=False):
    """bf16 decode of the packed state into `out` (concord/packed_b.py:158-170;
    consolidated=True drops s_fast as consolidated_weight does, 1632-1649)."""
    N, K = _check_packed(packed_w, row_exp, col_exp)
    assert out.dtype == torch.bfloat16 and tuple(out.shape) == (N, K) and out.stride(1) == 1
    C.check(C.lib().concord_materialize(
        C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp), C.ptr(col_exp), N, K,
        int(mantissa_bias), int(bool(consolidated)), C.ptr(out), out.stride(0),
        C.stream_of(packed_w.device)), "materialize_packed_bf16")
    return out


def apply_packed_sgd(packed_w, grad_W, weight_buf, row_exp, col_exp, row_max, col_max,
                     lr, mantissa_bias=15, alpha=0.1, beta1=0.0, alpha_v_fast=0.001,
                     mass_preserve=False, track_rebalance=True, salt_prebumped=False):
    """SGD update (concord/packed_b.py:362-394); weight_buf may be None (no emit)."""
    N, K = _check_packed(packed_w, row_exp, col_exp)
    assert grad_W.dtype == torch.bfloat16 and tuple(grad_W.shape) == (N, K) and grad_W.stride(1) == 1
    dev = packed_w.device
    flags = (C.MASS_PRESERVE if mass_preserve else 0) | (C.TRACK_REBALANCE if track_rebalance else 0)
    if weight_buf is not None:
        assert weight_buf.dtype == torch.bfloat16 and tuple(weight_buf.shape) == (N, K)
        flags |= C.EMIT_WEIGHT
    if salt_prebumped:
        flags |= C.SALT_PREBUMPED
    lr_t = _ensure_lr_tensor(lr, dev)
    C.check(C.lib().concord_apply_sgd(
        C.ptr(packed_w), packed_w.stride(0), C.ptr(grad_W), grad_W.stride(0),
        C.ptr(weight_buf), weight_buf.stride(0) if weight_buf is not None else K,
        C.ptr(row_exp), C.ptr(col_exp), C.ptr(row_max), C.ptr(col_max), N, K, C.ptr(lr_t),
        int(mantissa_bias), float(alpha), float(beta1), float(alpha_v_fast),
        C.ptr(_get_step_counter(dev)), flags, C.stream_of(dev)), "apply_packed_sgd")


def _adamw_flags(mass_preserve, apply_chase, track_rebalance, gf_trust_delta_sq, gf_consol,
                 coh_pre, emit):
    f = 0
    if mass_preserve:
        f |= C.MASS_PRESERVE
    if apply_chase:
        f |= C.APPLY_CHASE
    if track_rebalance:
        f |= C.TRACK_REBALANCE
    if gf_trust_delta_sq > 0:
        f |= C.GF_TRUST_REGION
    if gf_consol > 0:
        f |= C.GF_CONSOLIDATION
    if coh_pre is not None:
        f |= C.COHPRE
    if _USE_FIXED_COH:
        f |= C.FIXED_COH
    if _RATIO_COH:
        f |= C.RATIO_COH
    if emit:
        f |= C.EMIT_WEIGHT
    if _PROTO_SEMANTICS:
        f |= C.PROTO_CONSF
    return f


def _adamw_setup(dev, lr, mantissa_bias, alpha, beta1, weight_decay, eps, step_cap, v_scale, precond_p,
                 gf_consol, drift_cancel_C, alpha_v_fast, wd_sv, wd_sf, mass_preserve, apply_chase,
                 track_rebalance, gf_trust_delta_sq, coh_pre, emit, salt_prebumped, drive_muon):
    """(flags, UpdateParams, DeviceScalars) of the adamw update: the packed
    update's hyperparameters (concord/packed_b.py:863-951) and the device
    scalars it reads (lr, eps, floors, salt counter)."""
    flags = _adamw_flags(mass_preserve, apply_chase, track_rebalance, gf_trust_delta_sq,
                         gf_consol, coh_pre, emit)
    if salt_prebumped:
        flags |= C.SALT_PREBUMPED
    if drive_muon:
        flags |= C.MUON
    lr_t = _ensure_lr_tensor(lr, dev)
    eps_t = _ensure_eps_tensor(eps, dev)
    cf, lf = _ensure_floor_tensors(dev)
    P = C.UpdateParams(alpha=alpha, beta1=beta1, weight_decay=weight_decay, step_cap=step_cap,
                       v_scale=v_scale, precond_p=precond_p, gf_consol=gf_consol,
                       drift_cancel_C=drift_cancel_C, alpha_v_fast=alpha_v_fast, wd_sv=wd_sv,
                       wd_sf=wd_sf, gf_trust_delta_sq=gf_trust_delta_sq, gate_gain=_GATE_GAIN,
                       mantissa_bias=int(mantissa_bias))
    S = C.DeviceScalars(lr_t.data_ptr(), eps_t.data_ptr(), cf.data_ptr(), lf.data_ptr(),
                        _v_bc_buf(dev).data_ptr(), _get_step_counter(dev).data_ptr(),
                        _get_consolidate_flag(dev).data_ptr())
    return flags, P, S


def apply_packed_adamw(packed_w, grad_W, weight_buf, row_exp, col_exp, row_max, col_max,
                       lr, mantissa_bias=15, alpha=0.1, beta1=0.0, weight_decay=0.0, eps=1.0,
                       step_cap=10.0, v_scale=1.0, precond_p=0.5, gf_consol=0.0,
                       drift_cancel_C=None, alpha_v_fast=0.001, wd_sv=0.0, wd_sf=0.0,
                       mass_preserve=False, apply_chase=True, track_rebalance=True,
                       v_row=None, v_col=None, sum_v_inv=None, gf_trust_delta_sq=0.0,
                       coh_pre=None, salt_prebumped=False, drive_muon=False):
    """The packed optimizer update (concord/packed_b.py:863-951).  weight_buf may be
    None (fused-forward mode: no bf16 emit).  drive_muon: grad_W carries the
    Muon drive and the update uses it as the step (docs/MUON_IMPLEMENTATION.md:87-119)."""
    if drift_cancel_C is None:
        drift_cancel_C = compute_drift_cancel_C(alpha, alpha_v_fast, mass_preserve=mass_preserve)
    N, K = _check_packed(packed_w, row_exp, col_exp)
    assert grad_W.dtype == torch.bfloat16 and tuple(grad_W.shape) == (N, K) and grad_W.stride(1) == 1
    dev = packed_w.device
    # v-hat feeds the trust-region denominator (not under the Muon drive) and
    # the non-fixed coherence gate (docs/MUON_IMPLEMENTATION.md:75-80)
    use_vhat = ((gf_trust_delta_sq > 0 and not drive_muon)
                or (not _USE_FIXED_COH and (gf_consol > 0 or coh_pre is not None or _RATIO_COH)))
    if use_vhat:
        assert v_row is not None and v_col is not None and sum_v_inv is not None, \
            "gf_trust/gf_consol/coh_pre/ratio_coh require v_row, v_col, sum_v_inv"
    if weight_buf is not None:
        assert weight_buf.dtype == torch.bfloat16 and tuple(weight_buf.shape) == (N, K)
    if coh_pre is not None:
        assert coh_pre.dtype == torch.float32 and tuple(coh_pre.shape) == (N, K)
    flags, P, S = _adamw_setup(dev, lr, mantissa_bias, alpha, beta1, weight_decay, eps, step_cap, v_scale,
                               precond_p, gf_consol, drift_cancel_C, alpha_v_fast, wd_sv, wd_sf, mass_preserve,
                               apply_chase, track_rebalance, gf_trust_delta_sq, coh_pre,
                               weight_buf is not None, salt_prebumped, drive_muon)
    C.check(C.lib().concord_apply_adamw(
        C.ptr(packed_w), packed_w.stride(0), C.ptr(grad_W), grad_W.stride(0),
        C.ptr(weight_buf), weight_buf.stride(0) if weight_buf is not None else K,
        C.ptr(row_exp), C.ptr(col_exp), C.ptr(row_max), C.ptr(col_max),
        C.ptr(v_row), C.ptr(v_col), C.ptr(sum_v_inv),
        C.ptr(coh_pre), coh_pre.stride(0) if coh_pre is not None else K, N, K,
        ctypes.byref(P), ctypes.byref(S), flags, C.stream_of(dev)), "apply_packed_adamw")


def vhat_ema(grad_W, v_row, v_col, sum_v_inv, beta2=0.999, row_max=None, col_max=None,
             salt_counter=None):
    """v_row/v_col EMA of grad^2 and 1/sum(v_row) in place
    (concord/packed_b.py:1288-1303); optionally zeroes the watermarks and
    advances the salt counter for the update that follows."""
    C.require_device_tensor(grad_W, "grad_W")
    N, K = grad_W.shape
    ws = _workspace(grad_W.device, N, K)
    C.check(C.lib().concord_vhat_ema(
        C.ptr(grad_W), grad_W.stride(0), N, K, float(beta2), C.ptr(v_row), C.ptr(v_col),
        C.ptr(sum_v_inv), C.ptr(row_max), C.ptr(col_max), C.ptr(salt_counter), C.ptr(ws),
        ws.numel(), C.stream_of(grad_W.device)), "vhat_ema")


def _reb_stats_update(ws, N, K, mag):
    """Rebalance diagnostics (the counters of concord/packed_b.py:1161-1179)
    from this call's decisions: the decide kernel leaves its int32 ticks
    (+1 up, -1 down, 0) for the N rows and then the K columns at the start of
    the workspace scratch.  A word whose row and column ticks sum to -s
    (tick-down) has its int8 fields shifted left by s; it clips when its
    larger int8 magnitude before the call, `mag` (None without tick-down),
    exceeds 127 after the shift.  Host syncs; off by default."""
    t = ws[C.WS_SCRATCH:C.WS_SCRATCH + 4 * (N + K)].view(torch.int32)
    rt, ct = t[:N], t[N:]
    clip = 0
    if mag is not None:
        lsh = (-(rt[:, None] + ct[None, :])).clamp(min=0)
        clip = int(((mag << lsh) > 127).sum())
    _REB_STATS['calls'] += 1
    _REB_STATS['tickup_dim'] += int((rt > 0).sum() + (ct > 0).sum())
    _REB_STATS['tickdown_dim'] += int((rt < 0).sum() + (ct < 0).sum())
    _REB_STATS['dim_total'] += N + K
    _REB_STATS['clip_elems'] += clip
    _REB_STATS['elem_total'] += N * K


def rebalance_packed(packed_w, row_exp, col_exp, row_max, col_max, MAX_M=24000, EXP_MAX=7,
                     EXP_MIN=-8, seed_buf=None, allow_tickdown=False, row_hwm=None,
                     col_hwm=None, advance_seed=False):
    """Exponent ratchet (concord/packed_b.py:1129-1190): tick a row/column
    exponent up when its watermark exceeds MAX_M (down, if allowed, when the
    median int8 magnitude is <= 31), SR-shifting the words.  Like the
    reference, the seed is read, not advanced, unless advance_seed."""
    N, K = _check_packed(packed_w, row_exp, col_exp)
    if seed_buf is None:
        seed_buf = _ensure_reb_seed_tensor(packed_w.device)
    mag = None
    if _REB_STATS is not None and allow_tickdown:
        # the larger int8 field magnitude of each word before the shift
        mag = torch.maximum(((packed_w << 16) >> 24).abs(), ((packed_w << 24) >> 24).abs())
    ws = _workspace(packed_w.device, N, K)
    C.check(C.lib().concord_rebalance(
        C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp), C.ptr(col_exp), C.ptr(row_max),
        C.ptr(col_max), C.ptr(row_hwm), C.ptr(col_hwm), C.ptr(seed_buf), N, K, int(MAX_M),
        int(EXP_MAX), int(EXP_MIN), int(bool(allow_tickdown)), int(bool(advance_seed)),
        C.ptr(ws), ws.numel(), C.stream_of(packed_w.device)), "rebalance_packed")
    if _REB_STATS is not None:
        _reb_stats_update(ws, N, K, mag)


def load_packed(W, packed_w, row_exp, col_exp, exp_min=-8, exp_max=7, mantissa_bias=15,
                finetune=False):
    """fp32 weights -> packed state (concord/packed_b.py:1570-1603, 1816-1856)."""
    N, K = _check_packed(packed_w, row_exp, col_exp)
    W = W.to(device=packed_w.device, dtype=torch.float32).contiguous()
    assert tuple(W.shape) == (N, K)
    C.check(C.lib().concord_load_weights(
        C.ptr(W), W.stride(0), N, K, int(exp_min), int(exp_max), int(mantissa_bias),
        int(bool(finetune)), C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp),
        C.ptr(col_exp), C.stream_of(packed_w.device)), "load_weights")


# ---------------------------------------------------------------------------
# autograd Function (concord/packed_b.py:1197-1353)
# ---------------------------------------------------------------------------
# When set to a list, each backward appends a copy of its bf16 grad_W: lets a
# checker replay the update from the identical gradient.
_DEBUG_CAPTURE = None


def _gemm_fwd(x2, packed_w, row_exp, col_exp, mantissa_bias, bias, weight_buf):
    M, K = x2.shape
    N = (weight_buf if weight_buf is not None else packed_w).shape[0]
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x2.device)
    st = C.stream_of(x2.device)
    ws = _gemm_workspace(x2.device, M, N, K)
    if weight_buf is None:
        C.check(C.lib().concord_dqgemm_fwd(
            C.ptr(x2), x2.stride(0), C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp),
            C.ptr(col_exp), int(mantissa_bias), C.ptr(bias), C.ptr(y), y.stride(0), M, N, K,
            C.ptr(ws), ws.numel(), st), "dqgemm_fwd")
    else:
        C.check(C.lib().concord_gemm_bf16_fwd(
            C.ptr(x2), x2.stride(0), C.ptr(weight_buf), weight_buf.stride(0), C.ptr(bias),
            C.ptr(y), y.stride(0), M, N, K, C.ptr(ws), ws.numel(), st), "gemm_bf16_fwd")
    return y


def _gemm_dgrad(dy, packed_w, row_exp, col_exp, mantissa_bias, weight_buf):
    M, N = dy.shape
    K = (weight_buf if weight_buf is not None else packed_w).shape[1]
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dy.device)
    st = C.stream_of(dy.device)
    ws = _gemm_workspace(dy.device, M, N, K)
    if weight_buf is None:
        C.check(C.lib().concord_dqgemm_dgrad(
            C.ptr(dy), dy.stride(0), C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp),
            C.ptr(col_exp), int(mantissa_bias), C.ptr(dx), dx.stride(0), M, N, K,
            C.ptr(ws), ws.numel(), st), "dqgemm_dgrad")
    else:
        C.check(C.lib().concord_gemm_bf16_dgrad(
            C.ptr(dy), dy.stride(0), C.ptr(weight_buf), weight_buf.stride(0), C.ptr(dx),
            dx.stride(0), M, N, K, C.ptr(ws), ws.numel(), st), "gemm_bf16_dgrad")
    return dx


def _wgrad(dy, x2):
    M, N = dy.shape
    K = x2.shape[1]
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=dy.device)
    ws = _gemm_workspace(dy.device, M, N, K)
    C.check(C.lib().concord_wgrad(C.ptr(dy), dy.stride(0), C.ptr(x2), x2.stride(0), C.ptr(gw),
                                  gw.stride(0), M, N, K, C.ptr(ws), ws.numel(),
                                  C.stream_of(dy.device)), "wgrad")
    return gw


def _wgrad_vhat(dy, x2, v_row, v_col, sum_v_inv, beta2, row_max, col_max, salt_counter,
                with_bias=False):
    """wgrad with the v-hat partials formed in its epilogue, then the EMA
    (concord/packed_b.py:1269-1303); same results as _wgrad + vhat_ema.
    with_bias: also returns grad_y.sum(0) (1338-1340), formed from the same
    dy fragments.  Returns (grad_W, grad_bias or None)."""
    M, N = dy.shape
    K = x2.shape[1]
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=dy.device)
    gb = torch.empty(N, dtype=torch.bfloat16, device=dy.device) if with_bias else None
    gws = _gemm_workspace(dy.device, M, N, K)
    ws = _workspace(dy.device, N, K, M if with_bias else 0)
    C.check(C.lib().concord_wgrad_vhat(
        C.ptr(dy), dy.stride(0), C.ptr(x2), x2.stride(0), C.ptr(gw), gw.stride(0), M, N, K,
        float(beta2), C.ptr(v_row), C.ptr(v_col), C.ptr(sum_v_inv), C.ptr(row_max), C.ptr(col_max),
        C.ptr(salt_counter), C.ptr(gb), C.ptr(ws), ws.numel(), C.ptr(gws), gws.numel(),
        C.stream_of(dy.device)), "wgrad_vhat")
    return gw, gb


def _dgrad_wgrad_vhat(dy, x2, packed_w, row_exp, col_exp, mantissa_bias, v_row, v_col, sum_v_inv,
                      beta2, row_max, col_max, salt_counter, with_bias=False):
    """_gemm_dgrad then _wgrad_vhat in one entry (concord_dgrad_wgrad_vhat):
    the dgrad's split-K reduction runs on the CUs the WGRAD grid leaves idle.
    Same results as the two calls.  Returns (grad_x, grad_W, grad_bias or None)."""
    M, N = dy.shape
    K = x2.shape[1]
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dy.device)
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=dy.device)
    gb = torch.empty(N, dtype=torch.bfloat16, device=dy.device) if with_bias else None
    gws = _gemm_workspace(dy.device, M, N, K)
    ws = _workspace(dy.device, N, K, M if with_bias else 0)
    C.check(C.lib().concord_dgrad_wgrad_vhat(
        C.ptr(dy), dy.stride(0), C.ptr(packed_w), packed_w.stride(0), C.ptr(row_exp), C.ptr(col_exp),
        int(mantissa_bias), C.ptr(dx), dx.stride(0), C.ptr(x2), x2.stride(0), C.ptr(gw), gw.stride(0),
        M, N, K, float(beta2), C.ptr(v_row), C.ptr(v_col), C.ptr(sum_v_inv), C.ptr(row_max),
        C.ptr(col_max), C.ptr(salt_counter), C.ptr(gb), C.ptr(ws), ws.numel(), C.ptr(gws), gws.numel(),
        C.stream_of(dy.device)), "dgrad_wgrad_vhat")
    return dx, gw, gb


# whether the last _dgrad_wgrad_update call took the combined launch
_LAST_FUSED = [0]


def _dgrad_wgrad_update(ctx, dy, x2, fuse=False):
    """_dgrad_wgrad_vhat followed by the adamw update of _packed_step, in one
    entry (concord_dgrad_wgrad_update, same results)
    (concord/packed_b.py:1263-1327, 1338-1340).  fuse: for the update's two
    fast flag sets the v-hat finalize and the update run in the WGRAD launch,
    from its tiles' accumulators.  Returns (grad_x, grad_bias or None)."""
    M, N = dy.shape
    K = x2.shape[1]
    dev = dy.device
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=dev)
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=dev)
    gb = torch.empty(N, dtype=torch.bfloat16, device=dev) if ctx.has_bias else None
    gws = _gemm_workspace(dev, M, N, K)
    ws = _workspace(dev, N, K, M if ctx.has_bias else 0)
    dcc = ctx.drift_cancel_C
    if dcc is None:
        dcc = compute_drift_cancel_C(ctx.alpha, ctx.alpha_v_fast, mass_preserve=ctx.mass_preserve)
    flags, P, S = _adamw_setup(dev, ctx.lr, ctx.mantissa_bias, ctx.alpha, ctx.beta1, ctx.weight_decay, ctx.eps,
                               ctx.step_cap, ctx.v_scale, ctx.precond_p, ctx.gf_consol, dcc, ctx.alpha_v_fast,
                               ctx.wd_sv, ctx.wd_sf, ctx.mass_preserve, ctx.apply_chase, ctx.track_rebalance,
                               ctx.gf_trust_delta_sq, ctx.coh_pre, False, True, False)
    rm = ctx.row_max_buf if ctx.track_rebalance else None
    cm = ctx.col_max_buf if ctx.track_rebalance else None
    cp = ctx.coh_pre
    capture = _DEBUG_CAPTURE is not None
    fused = ctypes.c_int(0)
    C.check(C.lib().concord_dgrad_wgrad_update(
        C.ptr(dy), dy.stride(0), C.ptr(ctx.packed_w), ctx.packed_w.stride(0), C.ptr(ctx.row_exp),
        C.ptr(ctx.col_exp), C.ptr(dx), dx.stride(0), C.ptr(x2), x2.stride(0), C.ptr(gw), gw.stride(0),
        int(capture), int(bool(fuse)), M, N, K, float(ctx.adafactor_beta2), C.ptr(ctx.v_row), C.ptr(ctx.v_col),
        C.ptr(ctx.sum_v_inv), C.ptr(rm), C.ptr(cm), C.ptr(cp), cp.stride(0) if cp is not None else K, C.ptr(gb),
        ctypes.byref(P), ctypes.byref(S), flags, C.ptr(ws), ws.numel(), C.ptr(gws), gws.numel(),
        ctypes.byref(fused), C.stream_of(dev)), "dgrad_wgrad_update")
    _LAST_FUSED[0] = fused.value
    if capture:
        _DEBUG_CAPTURE.append(gw.clone())
    return dx, gb


def wgrad_update_faults(device):
    """Reads and clears the fault flag of the combined backward launch on this
    device's workspace (synchronises): True when a launch since the last read
    gave up a grid-barrier wait and skipped its writes."""
    dev = torch.device(device)
    ws = _workspace(dev, 1, 1, 0)
    f = ctypes.c_int(0)
    C.check(C.lib().concord_wgrad_update_fault(C.ptr(ws), ws.numel(), ctypes.byref(f), C.stream_of(dev)),
            "wgrad_update_fault")
    return f.value != 0


_MUON_WORKSPACES = {}


def muon_ns5(grad_W, out=None, gamma=None):
    """The Muon drive O = bf16(gamma NS5(grad_W / ||grad_W||_F)), gamma =
    sqrt(max(N, K)) (experiments/cpu_dynamics/exp9_muon.py:44-55, 58-100;
    docs/MUON_IMPLEMENTATION.md:27-40)."""
    C.require_device_tensor(grad_W, "grad_W")
    assert grad_W.dtype == torch.bfloat16 and grad_W.dim() == 2 and grad_W.stride(1) == 1
    N, K = grad_W.shape
    if gamma is None:
        gamma = math.sqrt(max(N, K))
    if out is None:
        out = torch.empty((N, K), dtype=torch.bfloat16, device=grad_W.device)
    key = _dev_key(grad_W.device)
    need = int(C.lib().concord_muon_workspace_bytes(N, K))
    ws = _MUON_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=key)
        _MUON_WORKSPACES[key] = ws
    C.check(C.lib().concord_muon_ns5(C.ptr(grad_W), grad_W.stride(0), N, K, float(gamma), C.ptr(out),
                                     out.stride(0), C.ptr(ws), ws.numel(),
                                     C.stream_of(grad_W.device)), "muon_ns5")
    return out


def _bias_grad(dy):
    M, N = dy.shape
    need = int(C.lib().concord_workspace_bytes(N, 1, M))
    scratch = torch.empty(need, dtype=torch.uint8, device=dy.device)
    out = torch.empty(N, dtype=torch.bfloat16, device=dy.device)
    C.check(C.lib().concord_bias_grad(C.ptr(dy), dy.stride(0), M, N, C.ptr(out), C.ptr(scratch),
                                      scratch.numel(), C.stream_of(dy.device)), "bias_grad")
    return out


def _stash_step_args(ctx, layer, wbuf, rmbuf, cmbuf):
    """The optimizer arguments the module passes to FusedConcordLinearPackedB
    (ConcordLinearPackedB.forward), stored on ctx for _packed_step."""
    ctx.packed_w, ctx.row_exp, ctx.col_exp = layer.packed_w, layer.row_exp, layer.col_exp
    ctx.lr, ctx.alpha, ctx.beta1, ctx.mantissa_bias = layer._lr_buf, layer.alpha, layer.beta1, layer.MANTISSA_BIAS
    ctx.optimizer_kind = layer.optimizer_kind
    ctx.weight_decay, ctx.eps, ctx.step_cap = layer.weight_decay, layer._eps_buf, layer.step_cap
    ctx.v_scale, ctx.precond_p, ctx.gf_consol = layer.v_scale, layer.precond_p, layer.gf_consol
    ctx.drift_cancel_C, ctx.alpha_v_fast = layer.drift_cancel_C, layer.alpha_v_fast
    ctx.wd_sv, ctx.wd_sf = layer.wd_sv, layer.wd_sf
    ctx.mass_preserve, ctx.apply_chase = layer.mass_preserve_v, layer.apply_chase
    ctx.track_rebalance = layer.track_rebalance
    ctx.weight_buf, ctx.row_max_buf, ctx.col_max_buf = wbuf, rmbuf, cmbuf
    ctx.v_row, ctx.v_col, ctx.sum_v_inv = layer.v_row, layer.v_col, layer._sum_v_inv
    ctx.adafactor_beta2, ctx.track_adafactor_v = float(layer.adafactor_beta2), bool(layer.track_adafactor_v)
    ctx.gf_trust_delta_sq, ctx.coh_pre = float(layer.gf_trust_delta_sq), layer._coh_pre


def _packed_step(ctx, grad_W, prebumped, muon):
    """The optimizer step of a packed layer's backward from its bf16 grad_W
    (concord/packed_b.py:1281-1336): watermark zeroing unless the v-hat entry
    already did it, then the adamw or sgd update of the packed words."""
    if _DEBUG_CAPTURE is not None:
        _DEBUG_CAPTURE.append(grad_W.clone())
    if not prebumped and ctx.track_rebalance:
        ctx.row_max_buf.zero_()
        ctx.col_max_buf.zero_()
    if ctx.optimizer_kind == 'adamw':
        apply_packed_adamw(
            ctx.packed_w, grad_W, ctx.weight_buf, ctx.row_exp, ctx.col_exp,
            ctx.row_max_buf, ctx.col_max_buf, lr=ctx.lr, mantissa_bias=ctx.mantissa_bias,
            alpha=ctx.alpha, beta1=ctx.beta1, weight_decay=ctx.weight_decay, eps=ctx.eps,
            step_cap=ctx.step_cap, v_scale=ctx.v_scale, precond_p=ctx.precond_p,
            gf_consol=ctx.gf_consol, drift_cancel_C=ctx.drift_cancel_C,
            alpha_v_fast=ctx.alpha_v_fast, wd_sv=ctx.wd_sv, wd_sf=ctx.wd_sf,
            mass_preserve=ctx.mass_preserve, apply_chase=ctx.apply_chase,
            track_rebalance=ctx.track_rebalance, v_row=ctx.v_row, v_col=ctx.v_col,
            sum_v_inv=ctx.sum_v_inv, gf_trust_delta_sq=ctx.gf_trust_delta_sq,
            coh_pre=ctx.coh_pre, salt_prebumped=prebumped, drive_muon=muon)
    else:
        apply_packed_sgd(
            ctx.packed_w, grad_W, ctx.weight_buf, ctx.row_exp, ctx.col_exp,
            ctx.row_max_buf, ctx.col_max_buf, lr=ctx.lr, mantissa_bias=ctx.mantissa_bias,
            alpha=ctx.alpha, beta1=ctx.beta1, alpha_v_fast=ctx.alpha_v_fast,
            mass_preserve=ctx.mass_preserve, track_rebalance=ctx.track_rebalance,
            salt_prebumped=prebumped)


class FusedConcordLinearPackedB(torch.autograd.Function):
    """Linear forward; backward = dgrad + wgrad + v-hat EMA + packed update.
    Same 33 forward arguments as the reference (concord/packed_b.py:1201-1211).
    weight_buf = None selects the fused dequant-GEMM mode."""

    @staticmethod
    def forward(ctx, x, packed_w, row_exp, col_exp, bias,
                lr, alpha, beta1, mantissa_bias,
                optimizer_kind,
                weight_decay, eps, step_cap,
                v_scale, precond_p, gf_consol, drift_cancel_C, alpha_v_fast,
                wd_sv, wd_sf,
                mass_preserve, apply_chase, track_rebalance,
                weight_buf, row_max_buf, col_max_buf,
                v_row, v_col, sum_v_inv,
                adafactor_beta2, track_adafactor_v,
                gf_trust_delta_sq, coh_pre, *extra):
        # extra[0] (optional): the drive, 'vhat' (the reference's) or 'muon'
        # (docs/MUON_IMPLEMENTATION.md:56-67)
        ctx.n_extra = len(extra)
        ctx.drive = extra[0] if extra else 'vhat'
        K = packed_w.shape[1]
        lead = x.shape[:-1]
        x2 = x.reshape(-1, K)
        if x2.dtype != torch.bfloat16:
            x2 = x2.to(torch.bfloat16)
        x2 = x2.contiguous()
        bias_bf16 = None
        if bias is not None:
            bias_bf16 = bias if bias.dtype == torch.bfloat16 else bias.to(torch.bfloat16)
            bias_bf16 = bias_bf16.contiguous()
        y = _gemm_fwd(x2, packed_w, row_exp, col_exp, mantissa_bias, bias_bf16, weight_buf)
        ctx.save_for_backward(x2)
        ctx.lead = lead
        ctx.packed_w, ctx.row_exp, ctx.col_exp = packed_w, row_exp, col_exp
        ctx.lr, ctx.alpha, ctx.beta1, ctx.mantissa_bias = lr, alpha, beta1, mantissa_bias
        ctx.optimizer_kind = optimizer_kind
        ctx.weight_decay, ctx.eps, ctx.step_cap = weight_decay, eps, step_cap
        ctx.v_scale, ctx.precond_p, ctx.gf_consol = v_scale, precond_p, gf_consol
        ctx.drift_cancel_C, ctx.alpha_v_fast = drift_cancel_C, alpha_v_fast
        ctx.wd_sv, ctx.wd_sf = wd_sv, wd_sf
        ctx.mass_preserve, ctx.apply_chase = mass_preserve, apply_chase
        ctx.track_rebalance = track_rebalance
        ctx.has_bias = bias is not None
        ctx.weight_buf, ctx.row_max_buf, ctx.col_max_buf = weight_buf, row_max_buf, col_max_buf
        ctx.v_row, ctx.v_col, ctx.sum_v_inv = v_row, v_col, sum_v_inv
        ctx.adafactor_beta2, ctx.track_adafactor_v = adafactor_beta2, track_adafactor_v
        ctx.gf_trust_delta_sq, ctx.coh_pre = gf_trust_delta_sq, coh_pre
        return y.reshape(*lead, y.shape[-1])

    @staticmethod
    def backward(ctx, grad_y):
        (x2,) = ctx.saved_tensors
        N, K = ctx.packed_w.shape
        dy = grad_y.reshape(-1, N)
        if dy.dtype != torch.bfloat16:
            dy = dy.to(torch.bfloat16)
        dy = dy.contiguous()
        dev = dy.device
        salt = _get_step_counter(dev)
        prebumped = False
        grad_bias = None
        muon = ctx.drive == 'muon' and ctx.optimizer_kind == 'adamw'
        vhat = ctx.track_adafactor_v and ctx.v_row is not None
        if _SIGMAG_NOISE and muon:
            # the Muon drive's fluctuation is post-NS and isotropic,
            # O <- O + sigma ||O|| xi / ||xi|| (docs/MUON_IMPLEMENTATION.md:21,
            # 64-66): NS5 of the clean gradient, then the draw scaled to O
            grad_x = _gemm_dgrad(dy, ctx.packed_w, ctx.row_exp, ctx.col_exp, ctx.mantissa_bias,
                                 ctx.weight_buf).reshape(*ctx.lead, K)
            grad_W = muon_ns5(_wgrad(dy, x2))
            iso_noise_(grad_W, salt_counter=salt)
        elif _SIGMAG_NOISE:
            # noise enters grad_W before the v-hat EMA and the update
            # (prototype_packed_b.py:1484-1501): the products in turn, the
            # injection, then the standalone v-hat entry
            grad_x = _gemm_dgrad(dy, ctx.packed_w, ctx.row_exp, ctx.col_exp, ctx.mantissa_bias,
                                 ctx.weight_buf).reshape(*ctx.lead, K)
            grad_W = _wgrad(dy, x2)
            if _SIGMAG_ISO:
                iso_noise_(grad_W, salt_counter=salt)
            else:
                sigmag_noise_(grad_W, dy, x2, salt_counter=salt)
            if vhat:
                vhat_ema(grad_W, ctx.v_row, ctx.v_col, ctx.sum_v_inv, ctx.adafactor_beta2,
                         ctx.row_max_buf if ctx.track_rebalance else None,
                         ctx.col_max_buf if ctx.track_rebalance else None, salt)
                prebumped = True
        elif vhat and not muon and ctx.weight_buf is None:
            # dgrad on the pre-update weight (1263), wgrad (1269-1277), watermark
            # zeroing (1281-1283), v-hat EMA (1288-1303), salt + 1 (910-911) and
            # grad_y.sum(0) (1338-1340) in one entry
            if ctx.optimizer_kind == 'adamw':
                # ... and the update (1281-1327) in the same entry: the
                # separate launches, or with set_fused_update the finalize and
                # update inside the WGRAD launch
                grad_x, grad_bias = _dgrad_wgrad_update(ctx, dy, x2, _FUSED_UPDATE)
                grad_W = None
            else:
                grad_x, grad_W, grad_bias = _dgrad_wgrad_vhat(
                    dy, x2, ctx.packed_w, ctx.row_exp, ctx.col_exp, ctx.mantissa_bias, ctx.v_row, ctx.v_col,
                    ctx.sum_v_inv, ctx.adafactor_beta2, ctx.row_max_buf if ctx.track_rebalance else None,
                    ctx.col_max_buf if ctx.track_rebalance else None, salt, with_bias=ctx.has_bias)
            grad_x = grad_x.reshape(*ctx.lead, K)
            prebumped = True
        else:
            # dgrad on the pre-update weight (1263), before the update below
            grad_x = _gemm_dgrad(dy, ctx.packed_w, ctx.row_exp, ctx.col_exp, ctx.mantissa_bias,
                                 ctx.weight_buf).reshape(*ctx.lead, K)
            if muon:
                # O = sqrt(max(N, K)) NS5(grad_W / ||grad_W||); no v-hat
                # (docs/MUON_IMPLEMENTATION.md:45-67)
                grad_W = muon_ns5(_wgrad(dy, x2))
            elif vhat:
                # wgrad (1269-1277), watermark zeroing (1281-1283), v-hat EMA
                # (1288-1303), salt + 1 (910-911)
                grad_W, grad_bias = _wgrad_vhat(dy, x2, ctx.v_row, ctx.v_col, ctx.sum_v_inv,
                                                ctx.adafactor_beta2,
                                                ctx.row_max_buf if ctx.track_rebalance else None,
                                                ctx.col_max_buf if ctx.track_rebalance else None, salt,
                                                with_bias=ctx.has_bias)
                prebumped = True
            else:
                grad_W = _wgrad(dy, x2)
        if grad_W is not None:
            _packed_step(ctx, grad_W, prebumped, muon)
        if ctx.has_bias and grad_bias is None:
            grad_bias = _bias_grad(dy)
        return (grad_x, None, None, None, grad_bias,
                None, None, None, None,
                None,
                None, None, None,
                None, None, None, None, None,
                None, None,
                None, None, None,
                None, None, None,
                None, None, None,
                None, None, None, None) + (None,) * ctx.n_extra


# ---------------------------------------------------------------------------
# nn.Module (concord/packed_b.py:1356-1856)
# ---------------------------------------------------------------------------
class ConcordLinearPackedB(nn.Module):
    """int32 packed weight (int16 s_fast + int8x128 s_slow + int8x128 v_slow) on
    shared row/column exponents; the optimizer step runs in backward.

    Defaults = the reference's validated production optimizer: adamw, rank-1
    v-hat (v_scale=0, gf_trust_delta_sq=1, eps=1e-10, precond_p=0.5), fixed
    coherence gate with coh_pre allocated.  Extra argument: weight_cache
    (False = fused dequant-GEMM forward/dgrad, no bf16 weight copy)."""

    MANTISSA_BIAS = 15
    EXP_MIN = -8
    EXP_MAX = 7
    MAX_M = 24000

    def __init__(self, in_features, out_features, bias=True, device='cuda', alpha=0.1,
                 beta1=0.0, lr=0.01, weight_cache=False, drive='vhat'):
        super().__init__()
        device = torch.device(device)
        if device.type != 'cuda':
            raise RuntimeError(
                "concord_amd.ConcordLinearPackedB runs on a ROCm GPU; got device "
                f"{device}.  There is no CPU implementation of the packed path.")
        C.lib()
        self.in_features = in_features
        self.out_features = out_features
        self.alpha = alpha
        self.beta1 = beta1
        self.weight_cache = bool(weight_cache)
        self.set_drive(drive)
        self._lr_value = float(lr)
        self.optimizer_kind = 'adamw'
        self.weight_decay = 0.0
        self._eps_value = 1e-10
        self.step_cap = 10.0
        self.v_scale = 0.0
        self.precond_p = 0.5
        self.gf_consol = 0.0
        self._coh_pre = None
        self.fast_gain = 1.0
        self.alpha_v_fast = 0.001
        self.drift_cancel_C = compute_drift_cancel_C(alpha, self.alpha_v_fast, mass_preserve=True)
        self.track_adafactor_v = True
        self.adafactor_beta2 = 0.999
        self.gf_trust_delta_sq = 1.0
        self.allow_tickdown = False
        self.wd_sv = 0.0
        self.wd_sf = 0.0
        self.mass_preserve_v = True
        self.apply_chase = True
        self.track_rebalance = True
        self.register_buffer('_reb_seed', torch.zeros(1, dtype=torch.int32, device=device))
        self.register_buffer('packed_w', torch.zeros(out_features, in_features, dtype=torch.int32,
                                                     device=device))
        self.register_buffer('row_exp', torch.zeros(out_features, dtype=torch.int8, device=device))
        self.register_buffer('col_exp', torch.zeros(in_features, dtype=torch.int8, device=device))
        self.register_buffer('v_row', torch.zeros(out_features, dtype=torch.float32, device=device))
        self.register_buffer('v_col', torch.zeros(in_features, dtype=torch.float32, device=device))
        self.register_buffer('_sum_v_inv', torch.ones(1, dtype=torch.float32, device=device))
        self._coh_pre = torch.ones_like(self.packed_w, dtype=torch.float32)
        self.register_buffer('_row_max_hwm', torch.zeros(out_features, dtype=torch.int32,
                                                         device=device))
        self.register_buffer('_col_max_hwm', torch.zeros(in_features, dtype=torch.int32,
                                                         device=device))
        self.register_buffer('_lr_buf', torch.full((1,), self._lr_value, dtype=torch.float32,
                                                   device=device))
        self.register_buffer('_eps_buf', torch.full((1,), self._eps_value, dtype=torch.float32,
                                                    device=device))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16, device=device))
        else:
            self.register_parameter('bias', None)
        _workspace(device, out_features, in_features)
        self._init_weight()
        self._ensure_buffers()

    # -- properties (concord/packed_b.py:1500-1537) --
    @property
    def weight(self):
        """bf16 weight for code that inspects nn.Linear.weight.  With
        weight_cache=True this is the live buffer the update keeps fresh; in
        the fused mode it is a snapshot decoded on each access."""
        wbuf = getattr(self, '_bf16_weight_buf', None)
        if wbuf is not None:
            return wbuf
        return self.get_weight()

    @property
    def lr(self):
        return self._lr_value

    @lr.setter
    def lr(self, value):
        v = float(value)
        self._lr_value = v
        buf = getattr(self, '_lr_buf', None)
        if buf is not None:
            buf.fill_(v)

    @property
    def eps(self):
        return self._eps_value

    @eps.setter
    def eps(self, value):
        v = float(value)
        self._eps_value = v
        buf = getattr(self, '_eps_buf', None)
        if buf is not None:
            buf.fill_(v)

    # -- knobs (concord/packed_b.py:1539-1568) --
    @torch.no_grad()
    def enable_cohpre(self):
        self._coh_pre = torch.ones_like(self.packed_w, dtype=torch.float32)
        return self._coh_pre

    @torch.no_grad()
    def disable_cohpre(self):
        self._coh_pre = None

    def set_drive(self, drive):
        """'vhat' (default: clip(g / sqrt(v-hat + eps))) or 'muon' (the step is
        sqrt(max(N, K)) NS5(grad / ||grad||); no v-hat, eps or cap), after
        docs/MUON_IMPLEMENTATION.md:56-67."""
        if drive not in ('vhat', 'muon'):
            raise ValueError("drive must be 'vhat' or 'muon'")
        self.drive = drive

    def set_optimizer_kind(self, kind, weight_decay=0.0, eps=1.0, step_cap=10.0):
        if kind not in ('sgd', 'adamw'):
            raise ValueError("optimizer kind must be 'sgd' or 'adamw'")
        self.optimizer_kind = kind
        self.weight_decay = float(weight_decay)
        self.eps = float(eps)
        self.step_cap = float(step_cap)

    def _init_weight(self):
        std = (2.0 / (self.in_features + self.out_features)) ** 0.5
        w = torch.randn(self.out_features, self.in_features, device=self.packed_w.device) * std
        self.load_weights(w)

    @torch.no_grad()
    def load_weights(self, W):
        """Whole mantissa into s_fast, row exponents from the row max
        (concord/packed_b.py:1570-1603)."""
        load_packed(W, self.packed_w, self.row_exp, self.col_exp, self.EXP_MIN, self.EXP_MAX,
                    self.MANTISSA_BIAS, finetune=False)
        self._resync_weight_buf()

    @torch.no_grad()
    def load_weights_finetune(self, W):
        """Zero-gradient steady state: half the mantissa in v_slow, the rest in
        s_slow, the residual in s_fast (concord/packed_b.py:1816-1856)."""
        load_packed(W, self.packed_w, self.row_exp, self.col_exp, self.EXP_MIN, self.EXP_MAX,
                    self.MANTISSA_BIAS, finetune=True)
        self._resync_weight_buf()

    @torch.no_grad()
    def _resync_weight_buf(self):
        wbuf = getattr(self, '_bf16_weight_buf', None)
        if wbuf is not None:
            materialize_packed_bf16(self.packed_w, self.row_exp, self.col_exp, wbuf,
                                    self.MANTISSA_BIAS)

    @torch.no_grad()
    def get_weight(self):
        """Live bf16 weight decoded from the packed state (1617-1630)."""
        out = torch.empty(self.packed_w.shape, dtype=torch.bfloat16, device=self.packed_w.device)
        return materialize_packed_bf16(self.packed_w, self.row_exp, self.col_exp, out,
                                       self.MANTISSA_BIAS)

    @torch.no_grad()
    def consolidated_weight(self):
        """Deploy weight (128 s_slow + 128 v_slow) * 2^exp, s_fast dropped (1632-1649)."""
        out = torch.empty(self.packed_w.shape, dtype=torch.bfloat16, device=self.packed_w.device)
        return materialize_packed_bf16(self.packed_w, self.row_exp, self.col_exp, out,
                                       self.MANTISSA_BIAS, consolidated=True)

    # -- checkpoint (the buffers registered above travel in state_dict as in
    # concord/packed_b.py:1445-1486; the extra state adds what the reference
    # loses on save: the device salt counter of the SR streams, the coh_pre
    # EMA, which is not a registered buffer, and the optimizer settings) --
    _CHECKPOINT_FORMAT = 1
    _CHECKPOINT_KNOBS = ('alpha', 'beta1', 'optimizer_kind', 'weight_decay', 'step_cap', 'v_scale',
                         'precond_p', 'gf_consol', 'fast_gain', 'alpha_v_fast', 'drift_cancel_C',
                         'track_adafactor_v', 'adafactor_beta2', 'gf_trust_delta_sq', 'allow_tickdown',
                         'wd_sv', 'wd_sf', 'mass_preserve_v', 'apply_chase', 'track_rebalance', 'drive')

    def get_extra_state(self):
        """Resume state beyond the registered buffers: the per-device salt
        counter (read back once, at save time), coh_pre and the optimizer
        settings.  Plain tensors and Python scalars only, so the checkpoint
        loads with torch.load(..., weights_only=True)."""
        dev = self.packed_w.device
        return {
            'format': self._CHECKPOINT_FORMAT,
            'salt_counter': int(_get_step_counter(dev).item()),
            'coh_pre': None if self._coh_pre is None else self._coh_pre.detach().clone(),
            'knobs': {k: getattr(self, k) for k in self._CHECKPOINT_KNOBS},
        }

    @torch.no_grad()
    def set_extra_state(self, state):
        """Restore get_extra_state()'s record after the buffers have loaded:
        the device salt counter is set to the saved value (it is shared by the
        device's layers, which all saved the same value), lr / eps follow the
        loaded device scalars, and the bf16 weight copy is re-materialised."""
        if not isinstance(state, dict) or state.get('format') != self._CHECKPOINT_FORMAT:
            raise ValueError("ConcordLinearPackedB: unknown checkpoint extra-state format")
        dev = self.packed_w.device
        for k, v in state['knobs'].items():
            if k in self._CHECKPOINT_KNOBS:
                if k == 'drive':
                    self.set_drive(v)
                else:
                    setattr(self, k, v)
        cp = state['coh_pre']
        if cp is None:
            self._coh_pre = None
        else:
            if tuple(cp.shape) != tuple(self.packed_w.shape):
                raise ValueError("ConcordLinearPackedB: coh_pre shape does not match the layer")
            self._coh_pre = cp.to(device=dev, dtype=torch.float32).contiguous()
        _get_step_counter(dev).fill_(int(state['salt_counter']))
        self._lr_value = float(self._lr_buf.item())
        self._eps_value = float(self._eps_buf.item())
        self._resync_weight_buf()

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys,
                              unexpected_keys, error_msgs):
        """A state_dict without the extra-state entry (the reference class
        writes none: its keys are the registered buffers of
        concord/packed_b.py:1445-1492) loads under strict=True too: the salt
        counter and coh_pre keep their current values, lr / eps follow the
        loaded device scalars."""
        key = prefix + '_extra_state'
        absent = key not in state_dict
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys,
                                      unexpected_keys, error_msgs)
        if absent:
            while key in missing_keys:
                missing_keys.remove(key)
            if getattr(self, '_lr_buf', None) is not None and self._lr_buf.numel() == 1:
                self._lr_value = float(self._lr_buf.item())
                self._eps_value = float(self._eps_buf.item())
            self._resync_weight_buf()

    @torch.no_grad()
    def get_state(self):
        p = self.packed_w
        return p >> 16, (p << 16) >> 24, (p << 24) >> 24

    @torch.no_grad()
    def get_rebalance_watermark_stats(self):
        if getattr(self, '_row_max_buf', None) is None or not self.track_rebalance:
            return None, None
        return self._row_max_hwm.clone(), self._col_max_hwm.clone()

    @torch.no_grad()
    def get_garbage_fraction_stats(self):
        """Per-weight garbage fraction quantiles (diagnostic, 1676-1730)."""
        if float(self.v_row.sum().item()) <= 0.0:
            return None
        s_fast, s_slow, v_slow = (t.to(torch.float32) for t in self.get_state())
        noise = s_fast - float(self.drift_cancel_C) * (s_slow - v_slow) * 128.0
        exp = (self.row_exp[:, None].to(torch.float32) + self.col_exp[None, :].to(torch.float32)
               - self.MANTISSA_BIAS)
        var_W = (noise * torch.pow(2.0, exp)) ** 2
        sum_v = self.v_row.float().sum().clamp(min=1e-30)
        v_hat = self.v_row.float()[:, None] * self.v_col.float()[None, :] / sum_v
        flat = (var_W / (v_hat + 1e-30)).clamp(0.0, 1.0).flatten()
        q = torch.quantile(flat, torch.tensor([0.25, 0.5, 0.75], device=flat.device))
        return {'mean': flat.mean().item(), 'p25': q[0].item(), 'median': q[1].item(),
                'p75': q[2].item(),
                'frac_signal_dominated': (flat < 0.1).float().mean().item(),
                'frac_noise_dominated': (flat > 0.9).float().mean().item()}

    def _ensure_buffers(self):
        N, K = self.packed_w.shape
        dev = self.packed_w.device
        wbuf = getattr(self, '_bf16_weight_buf', None)
        if self.weight_cache and (wbuf is None or wbuf.shape != self.packed_w.shape):
            wbuf = torch.empty(self.packed_w.shape, dtype=torch.bfloat16, device=dev)
            self._bf16_weight_buf = wbuf
            materialize_packed_bf16(self.packed_w, self.row_exp, self.col_exp, wbuf,
                                    self.MANTISSA_BIAS)
        if not self.weight_cache:
            self._bf16_weight_buf = None
            wbuf = None
        rmbuf = getattr(self, '_row_max_buf', None)
        if rmbuf is None or rmbuf.shape[0] != N:
            self._row_max_buf = rmbuf = torch.zeros(N, dtype=torch.int32, device=dev)
        cmbuf = getattr(self, '_col_max_buf', None)
        if cmbuf is None or cmbuf.shape[0] != K:
            self._col_max_buf = cmbuf = torch.zeros(K, dtype=torch.int32, device=dev)
        return wbuf, rmbuf, cmbuf

    def forward(self, x):
        return self._forward_rows(x, self.fast_gain)

    def _forward_rows(self, x, fast_gain):
        """forward() on rows of features; fast_gain < 1 gates s_fast out of the
        forward weight (the linear layer's forward; the conv layer passes 1.0,
        since the reference's conv forward never gates, 2046-2065)."""
        in_dtype = x.dtype
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        wbuf, rmbuf, cmbuf = self._ensure_buffers()
        if fast_gain < 1.0:
            # gate s_fast out of the forward weight (1762-1772); the GEMMs then read
            # the gated bf16 copy, the packed state keeps the full s_fast
            pw = self.packed_w
            if wbuf is None:
                wbuf = torch.empty(pw.shape, dtype=torch.bfloat16, device=pw.device)
            C.check(C.lib().concord_materialize_gated(
                C.ptr(pw), pw.stride(0), C.ptr(self.row_exp), C.ptr(self.col_exp), pw.shape[0],
                pw.shape[1], self.MANTISSA_BIAS, float(fast_gain), C.ptr(wbuf), wbuf.stride(0),
                C.stream_of(pw.device)), "materialize_gated")
        y = FusedConcordLinearPackedB.apply(
            x, self.packed_w, self.row_exp, self.col_exp, self.bias,
            self._lr_buf, self.alpha, self.beta1, self.MANTISSA_BIAS,
            self.optimizer_kind,
            self.weight_decay, self._eps_buf, self.step_cap,
            self.v_scale, self.precond_p, self.gf_consol, self.drift_cancel_C, self.alpha_v_fast,
            self.wd_sv, self.wd_sf,
            self.mass_preserve_v, self.apply_chase, self.track_rebalance,
            wbuf, rmbuf, cmbuf,
            self.v_row, self.v_col, self._sum_v_inv,
            float(self.adafactor_beta2), bool(self.track_adafactor_v),
            float(self.gf_trust_delta_sq), self._coh_pre, self.drive)
        return y.to(in_dtype)

    @torch.no_grad()
    def rebalance(self):
        """Watermarks -> high-watermarks, seed + 1, exponent ratchet (1792-1814).
        Entirely on device; no host synchronisation."""
        rmbuf = getattr(self, '_row_max_buf', None)
        cmbuf = getattr(self, '_col_max_buf', None)
        if rmbuf is None or cmbuf is None:
            return
        rebalance_packed(self.packed_w, self.row_exp, self.col_exp, rmbuf, cmbuf,
                         MAX_M=self.MAX_M, EXP_MAX=self.EXP_MAX, EXP_MIN=self.EXP_MIN,
                         seed_buf=self._reb_seed, allow_tickdown=self.allow_tickdown,
                         row_hwm=self._row_max_hwm, col_hwm=self._col_max_hwm,
                         advance_seed=True)


# ---------------------------------------------------------------------------
# Gradient-noise injection (notebook/src/prototype_packed_b.py:876-916, 1472-1501)
# ---------------------------------------------------------------------------
_SIGMAG_NOISE = False
_SIGMAG_ISO = False
_SIGMAG_SIGMA = 0.0
_SIGMAG_SIGMA_T = {}
_NOISE_WORKSPACES = {}


def set_sigmag_noise(enabled, isotropic=False):
    """Turn the gradient-noise injection on or off (a Python switch: a
    captured graph keeps the choice made at capture, as in the reference).
    Default: the centred Sigma_g-shaped draw (eps * dy)^T x - (sum eps) g / M;
    isotropic=True: white noise.  Either is scaled to sigma ||grad_W||.
    Layers with drive='muon' always take the isotropic draw after NS5,
    scaled to sigma ||O|| (docs/MUON_IMPLEMENTATION.md:21, 64-66)."""
    global _SIGMAG_NOISE, _SIGMAG_ISO
    _SIGMAG_NOISE = bool(enabled)
    _SIGMAG_ISO = bool(isotropic)


def set_sigmag_sigma(sigma):
    """Noise magnitude in units of ||grad_W||: the Python value and every
    device-tensor copy (filled in place, so graph replays see it)."""
    global _SIGMAG_SIGMA
    _SIGMAG_SIGMA = float(sigma)
    for t in _SIGMAG_SIGMA_T.values():
        t.fill_(_SIGMAG_SIGMA)


def _get_sigmag_sigma(device):
    key = _dev_key(device)
    t = _SIGMAG_SIGMA_T.get(key)
    if t is None:
        t = torch.full((1,), _SIGMAG_SIGMA, dtype=torch.float32, device=key)
        _SIGMAG_SIGMA_T[key] = t
    return t


_SIGMAG_WORKSPACES = {}


def sigmag_noise_(grad_W, dy, x2, sigma=None, salt_counter=None):
    """grad_W <- bf16(g + n sigma ||g|| / max(||n||, 1e-12)) in place with the
    centred Sigma_g-shaped draw n = (eps * dy)^T x - (sum eps) g / M
    (prototype_packed_b.py:1489-1500; concord_sigmag_noise); eps_m is the
    library's per-token normal stream keyed by the salt counter (read, not
    advanced), and the product runs on the WGRAD kernels."""
    C.require_device_tensor(grad_W, "grad_W")
    N, K = grad_W.shape
    M = dy.shape[0]
    dev = grad_W.device
    if sigma is None:
        sigma = _get_sigmag_sigma(dev)
    if salt_counter is None:
        salt_counter = _get_step_counter(dev)
    key = _dev_key(dev)
    need = int(C.lib().concord_sigmag_noise_workspace_bytes(M, N, K))
    ws = _SIGMAG_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=key)
        _SIGMAG_WORKSPACES[key] = ws
    C.check(C.lib().concord_sigmag_noise(C.ptr(grad_W), grad_W.stride(0), C.ptr(dy), dy.stride(0), C.ptr(x2),
                                         x2.stride(0), M, N, K, C.ptr(sigma), C.ptr(salt_counter), C.ptr(ws),
                                         ws.numel(), C.stream_of(dev)), "sigmag_noise")
    return grad_W


def iso_noise_(grad_W, sigma=None, salt_counter=None):
    """grad_W <- bf16(g + xi sigma ||g|| / max(||xi||, 1e-12)) in place
    (concord_iso_noise); xi is the library's counter-based normal stream keyed
    by the device salt counter (read, not advanced)."""
    C.require_device_tensor(grad_W, "grad_W")
    N, K = grad_W.shape
    dev = grad_W.device
    if sigma is None:
        sigma = _get_sigmag_sigma(dev)
    if salt_counter is None:
        salt_counter = _get_step_counter(dev)
    key = _dev_key(dev)
    need = int(C.lib().concord_noise_workspace_bytes(N, K))
    ws = _NOISE_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=key)
        _NOISE_WORKSPACES[key] = ws
    C.check(C.lib().concord_iso_noise(C.ptr(grad_W), grad_W.stride(0), N, K, C.ptr(sigma),
                                      C.ptr(salt_counter), C.ptr(ws), ws.numel(), C.stream_of(dev)),
            "iso_noise")
    return grad_W


# ---------------------------------------------------------------------------
# Conv2d on the packed path (concord/packed_b.py:1863-2065)
# ---------------------------------------------------------------------------
def _pair(v):
    return (int(v), int(v)) if isinstance(v, int) else (int(v[0]), int(v[1]))


class _Im2col(torch.autograd.Function):
    """(B, C, H, W) bf16 -> the (B * Ho * Wo, C * kh * kw) patch matrix in one
    HIP pass (concord_conv_im2col).  The adjoint gathers dx straight from the
    patch gradient (concord_conv_col2im: fixed order, fp32 accumulation)."""

    @staticmethod
    def forward(ctx, x, kh, kw, sh, sw, ph, pw):
        x = x.contiguous()
        B, Cin, H, W = x.shape
        Ho = (H + 2 * ph - kh) // sh + 1
        Wo = (W + 2 * pw - kw) // sw + 1
        cols = torch.empty((B * Ho * Wo, Cin * kh * kw), dtype=torch.bfloat16, device=x.device)
        C.check(C.lib().concord_conv_im2col(C.ptr(x), B, Cin, H, W, kh, kw, sh, sw, ph, pw, C.ptr(cols),
                                            C.stream_of(x.device)), "conv_im2col")
        ctx.geom = (B, Cin, H, W, kh, kw, sh, sw, ph, pw, Ho * Wo)
        return cols

    @staticmethod
    def backward(ctx, dcols):
        B, Cin, H, W, kh, kw, sh, sw, ph, pw, L = ctx.geom
        dcols = dcols.to(torch.bfloat16).contiguous()
        dx = torch.empty((B, Cin, H, W), dtype=torch.bfloat16, device=dcols.device)
        C.check(C.lib().concord_conv_col2im(C.ptr(dcols), B, Cin, H, W, kh, kw, sh, sw, ph, pw, C.ptr(dx),
                                            C.stream_of(dcols.device)), "conv_col2im")
        return dx, None, None, None, None, None, None


class _ToNCHW(torch.autograd.Function):
    """(B * L, N) rows in (b, ho, wo) order -> (B, N, Ho, Wo), the 1 x 1 case
    of concord_conv_col2im (a transpose through LDS); the adjoint is the 1 x 1
    im2col."""

    @staticmethod
    def forward(ctx, y2, B, Ho, Wo):
        y2 = y2.to(torch.bfloat16).contiguous()
        N = y2.shape[1]
        y = torch.empty((B, N, Ho, Wo), dtype=torch.bfloat16, device=y2.device)
        C.check(C.lib().concord_conv_col2im(C.ptr(y2), B, N, Ho, Wo, 1, 1, 1, 1, 0, 0, C.ptr(y),
                                            C.stream_of(y2.device)), "conv_col2im")
        ctx.shape = (B, N, Ho, Wo)
        return y

    @staticmethod
    def backward(ctx, dy):
        B, N, Ho, Wo = ctx.shape
        dy = dy.to(torch.bfloat16).contiguous()
        d2 = torch.empty((B * Ho * Wo, N), dtype=torch.bfloat16, device=dy.device)
        C.check(C.lib().concord_conv_im2col(C.ptr(dy), B, N, Ho, Wo, 1, 1, 1, 1, 0, 0, C.ptr(d2),
                                            C.stream_of(dy.device)), "conv_im2col")
        return d2, None, None, None


_CONV_WORKSPACES = {}


def _conv_workspace(device, geom):
    """Zero-initialised per-device split-K workspace of the implicit conv
    products, grown to the largest geometry seen."""
    key = _dev_key(device)
    need = int(C.lib().concord_conv_workspace_bytes(*geom))
    ws = _CONV_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.zeros(need, dtype=torch.uint8, device=key)
        _CONV_WORKSPACES[key] = ws
    return ws


def _nhwc(t):
    """(B, C, H, W) -> its channels-last storage viewed as (B, H, W, C)
    (no copy when t already is channels-last contiguous)."""
    if t.dtype != torch.bfloat16:
        t = t.to(torch.bfloat16)
    return t.contiguous(memory_format=torch.channels_last).permute(0, 2, 3, 1)


class FusedConcordConv2dImplicit(torch.autograd.Function):
    """Conv2d over the packed state by implicit GEMM on channels-last
    activations (FusedConcordConv2dPackedB, concord/packed_b.py:1863-2025,
    where the reference runs cuDNN on the cached bf16 weight).  Forward:
    W'[n][tap][c] decoded from the packed words (concord_conv_weight_taps),
    y = conv(x, W') + bias with the patches gathered inside the GEMM
    (concord_conv_fwd).  Backward: dx by the transposed gather
    (concord_conv_dgrad, on the pre-update W'), grad_W by the gathered WGRAD
    (concord_conv_wgrad) put back in (c, tap) order, then the layer's
    optimizer step (v-hat EMA, packed update), as the linear path takes it.
    Without the Muon drive or a noise draw, the WGRAD, the reorder, the v-hat
    EMA and the bias gradient are one entry (concord_conv_wgrad_vhat).
    The output and dx are channels-last NCHW tensors."""

    @staticmethod
    def forward(ctx, x, bias, layer, geom, wbuf, rmbuf, cmbuf):
        B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw = geom
        Ho = (H + 2 * ph - kh) // sh + 1
        Wo = (W + 2 * pw - kw) // sw + 1
        T = kh * kw
        dev = x.device
        st = C.stream_of(dev)
        x4 = _nhwc(x)
        pw_ = layer.packed_w
        wt = torch.empty((Cout, T * Cin), dtype=torch.bfloat16, device=dev)
        C.check(C.lib().concord_conv_weight_taps(
            C.ptr(pw_), pw_.stride(0), C.ptr(layer.row_exp), C.ptr(layer.col_exp), Cout, Cin, T,
            layer.MANTISSA_BIAS, 1.0, C.ptr(wt), st), "conv_weight_taps")
        bias_bf16 = None
        if bias is not None:
            bias_bf16 = (bias if bias.dtype == torch.bfloat16 else bias.to(torch.bfloat16)).contiguous()
        y2 = torch.empty((B * Ho * Wo, Cout), dtype=torch.bfloat16, device=dev)
        ws = _conv_workspace(dev, geom)
        C.check(C.lib().concord_conv_fwd(C.ptr(x4), C.ptr(wt), C.ptr(bias_bf16), C.ptr(y2), *geom, C.ptr(ws),
                                         ws.numel(), st), "conv_fwd")
        ctx.save_for_backward(x4, wt)
        ctx.geom, ctx.out_hw = geom, (Ho, Wo)
        ctx.drive = layer.drive
        ctx.has_bias = bias is not None
        _stash_step_args(ctx, layer, wbuf, rmbuf, cmbuf)
        return y2.view(B, Ho, Wo, Cout).permute(0, 3, 1, 2)

    @staticmethod
    def backward(ctx, grad_y):
        x4, wt = ctx.saved_tensors
        geom = ctx.geom
        B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw = geom
        Ho, Wo = ctx.out_hw
        T = kh * kw
        dy2 = _nhwc(grad_y).reshape(B * Ho * Wo, Cout)
        dev = dy2.device
        st = C.stream_of(dev)
        ws = _conv_workspace(dev, geom)
        grad_x = None
        if ctx.needs_input_grad[0]:
            dx = torch.empty((B, H, W, Cin), dtype=torch.bfloat16, device=dev)
            C.check(C.lib().concord_conv_dgrad(C.ptr(dy2), C.ptr(wt), C.ptr(dx), *geom, C.ptr(ws), ws.numel(),
                                               st), "conv_dgrad")
            grad_x = dx.permute(0, 3, 1, 2)
        gt = torch.empty((Cout, T * Cin), dtype=torch.bfloat16, device=dev)
        grad_W = torch.empty((Cout, Cin * T), dtype=torch.bfloat16, device=dev)
        salt = _get_step_counter(dev)
        muon = ctx.drive == 'muon' and ctx.optimizer_kind == 'adamw'
        vhat = ctx.track_adafactor_v and ctx.v_row is not None
        prebumped = False
        grad_bias = None
        if vhat and not muon and not _SIGMAG_NOISE:
            # product, reorder, v-hat EMA and bias gradient in one entry
            M = B * Ho * Wo
            gb = torch.empty(Cout, dtype=torch.bfloat16, device=dev) if ctx.has_bias else None
            wsu = _workspace(dev, Cout, Cin * T, M if ctx.has_bias else 0)
            rm = ctx.row_max_buf if ctx.track_rebalance else None
            cm = ctx.col_max_buf if ctx.track_rebalance else None
            C.check(C.lib().concord_conv_wgrad_vhat(
                C.ptr(dy2), C.ptr(x4), C.ptr(gt), C.ptr(grad_W), grad_W.stride(0), *geom,
                float(ctx.adafactor_beta2), C.ptr(ctx.v_row), C.ptr(ctx.v_col), C.ptr(ctx.sum_v_inv),
                C.ptr(rm), C.ptr(cm), C.ptr(salt), C.ptr(gb), C.ptr(wsu), wsu.numel(), C.ptr(ws), ws.numel(),
                st), "conv_wgrad_vhat")
            _packed_step(ctx, grad_W, True, False)
            return grad_x, gb, None, None, None, None, None
        C.check(C.lib().concord_conv_wgrad(C.ptr(dy2), C.ptr(x4), C.ptr(gt), *geom, C.ptr(ws), ws.numel(), st),
                "conv_wgrad")
        C.check(C.lib().concord_conv_grad_from_taps(C.ptr(gt), Cout, Cin, T, C.ptr(grad_W), grad_W.stride(0), st),
                "conv_grad_from_taps")
        if muon:
            grad_W = muon_ns5(grad_W)
        if _SIGMAG_NOISE:
            if not (muon or _SIGMAG_ISO):
                raise RuntimeError("ConcordConv2dPackedB: the Sigma_g noise draw was switched on between this "
                                   "layer's forward (implicit-GEMM path) and its backward")
            iso_noise_(grad_W, salt_counter=salt)
        if vhat and not muon:
            vhat_ema(grad_W, ctx.v_row, ctx.v_col, ctx.sum_v_inv, ctx.adafactor_beta2,
                     ctx.row_max_buf if ctx.track_rebalance else None,
                     ctx.col_max_buf if ctx.track_rebalance else None, salt)
            prebumped = True
        _packed_step(ctx, grad_W, prebumped, muon)
        grad_bias = _bias_grad(dy2) if ctx.has_bias else None
        return grad_x, grad_bias, None, None, None, None, None


class ConcordConv2dPackedB(ConcordLinearPackedB):
    """Conv2d variant of ConcordLinearPackedB (concord/packed_b.py:2028-2065):
    the same packed int32 state, an (out_channels, in_channels * kh * kw)
    matrix in nn.Conv2d's (c, i, j) flattening.  Where the reference runs
    cuDNN on the cached bf16 weight, this layer takes one of three HIP paths:
      * 1 x 1, stride 1, no padding: the linear layer's fused dequant-GEMM
        path on the channels-last positions (B * H * W, in_channels);
      * in and out channels multiples of 64, strides 1 or 2: implicit GEMM
        (FusedConcordConv2dImplicit) -- the patches are gathered inside the
        GEMM kernels from channels-last activations, no patch matrix;
      * otherwise (e.g. a 4-channel latent input): the patch matrix is
        gathered in one HIP pass (concord_conv_im2col), the linear path runs
        on it, and col2im gathers dx back (concord_conv_col2im).
    The first two return channels-last NCHW tensors."""

    def __init__(self, in_channels, out_channels, kernel_size, stride=1, padding=0, bias=True,
                 device='cuda', alpha=0.1, beta1=0.0, lr=0.01, weight_cache=False, drive='vhat'):
        kh, kw = _pair(kernel_size)
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kh, self.kw = kh, kw
        self.stride = stride
        self.padding = padding
        super().__init__(in_features=in_channels * kh * kw, out_features=out_channels, bias=bias,
                         device=device, alpha=alpha, beta1=beta1, lr=lr, weight_cache=weight_cache,
                         drive=drive)

    def _geom(self, x):
        B, cin, H, W = x.shape
        if cin != self.in_channels:
            raise ValueError(f"ConcordConv2dPackedB: expected {self.in_channels} input channels, "
                             f"got {cin}")
        (sh, sw), (ph, pw) = _pair(self.stride), _pair(self.padding)
        return (B, cin, H, W, self.out_channels, self.kh, self.kw, sh, sw, ph, pw)

    def conv_path(self, x):
        """'linear' (1 x 1), 'implicit' or 'im2col': the path forward(x) takes."""
        B, cin, H, W, cout, kh, kw, sh, sw, ph, pw = self._geom(x)
        if kh == kw == sh == sw == 1 and ph == pw == 0:
            return 'linear'
        # the Sigma_g noise draw needs the patch matrix
        sigmag = _SIGMAG_NOISE and not _SIGMAG_ISO and self.drive != 'muon'
        if not sigmag and C.lib().concord_conv_implicit_ok(B, cin, H, W, cout, kh, kw, sh, sw, ph, pw):
            return 'implicit'
        return 'im2col'

    def forward(self, x):
        if x.dim() != 4:
            raise ValueError("ConcordConv2dPackedB expects (B, C, H, W) input")
        in_dtype = x.dtype
        if x.dtype != torch.bfloat16:
            x = x.to(torch.bfloat16)
        geom = self._geom(x)
        B, cin, H, W, cout, kh, kw, sh, sw, ph, pw = geom
        path = self.conv_path(x)
        # the reference's conv forward (concord/packed_b.py:2046-2065) runs on
        # the ungated weight: fast_gain does not apply to convolutions
        if path == 'linear':
            x2 = _nhwc(x).reshape(B * H * W, cin)
            y = self._forward_rows(x2, 1.0).view(B, H, W, cout).permute(0, 3, 1, 2)
        elif path == 'implicit':
            wbuf, rmbuf, cmbuf = self._ensure_buffers()
            y = FusedConcordConv2dImplicit.apply(x, self.bias, self, geom, wbuf, rmbuf, cmbuf)
        else:
            Ho = (H + 2 * ph - kh) // sh + 1
            Wo = (W + 2 * pw - kw) // sw + 1
            cols = _Im2col.apply(x, kh, kw, sh, sw, ph, pw)
            y = _ToNCHW.apply(self._forward_rows(cols, 1.0), B, Ho, Wo)
        return y.to(in_dtype)

    @property
    def weight(self):
        """bf16 (out, in, kh, kw) weight, as nn.Conv2d.weight."""
        return ConcordLinearPackedB.weight.fget(self).view(self.out_channels, self.in_channels,
                                                          self.kh, self.kw)

    @torch.no_grad()
    def load_weights(self, W):
        """W: (out, in, kh, kw) or its (out, in * kh * kw) flattening."""
        super().load_weights(W.reshape(self.out_channels, -1))

    @torch.no_grad()
    def load_weights_finetune(self, W):
        super().load_weights_finetune(W.reshape(self.out_channels, -1))


# ---------------------------------------------------------------------------
# Multi-layer statistics: gated rebalance and the coherence meter
# (notebook/src/concord_winner.py:206-262, concord/packed_b.py:2081-2106)
# ---------------------------------------------------------------------------
_STATS_WORKSPACES = {}


def _stats_workspace(device, n_watermarks, n_words):
    key = _dev_key(device)
    need = int(C.lib().concord_stats_workspace_bytes(int(n_watermarks), int(n_words)))
    ws = _STATS_WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(need, dtype=torch.uint8, device=key)
        _STATS_WORKSPACES[key] = ws
    return ws


def gate_coherence_from_fields(s_fast, s_slow_i8, v_slow_i8, drift_cancel_C):
    """The update's FIXED_COH Wiener gain from unpacked integer fields given
    as float tensors (concord/packed_b.py:2081-2091); the exponents cancel.
    Elementwise tensor helper, as in the reference."""
    d_sv = (s_slow_i8 - v_slow_i8) * 128.0
    sig = drift_cancel_C * d_sv
    noise = s_fast - sig
    sig2 = sig * sig
    return sig2 / (sig2 + noise * noise + 1e-30)


@torch.no_grad()
def measure_coherence(layer):
    """Mean gate coherence of one Concord layer read from its packed words
    (concord/packed_b.py:2094-2106): one HIP reduction in a fixed order
    (concord_coherence_sum) and one host read of the sum."""
    p = layer.packed_w
    N, K = p.shape
    out = torch.empty(1, dtype=torch.float32, device=p.device)
    ws = _stats_workspace(p.device, 0, N * K)
    C.check(C.lib().concord_coherence_sum(C.ptr(p), p.stride(0), N, K, float(layer.drift_cancel_C),
                                          C.ptr(out), C.ptr(ws), ws.numel(), C.stream_of(p.device)),
            "coherence_sum")
    return float(out.item()) / float(max(N * K, 1))


class GatedRebalance:
    """Fire rebalance only when some layer's mantissa crosses MAX_M
    (notebook/src/concord_winner.py:206-262).  Every layer's row / column
    watermark buffers become slices of two shared slabs; one call is one HIP
    reduction over both slabs (concord_watermark_peak) followed by the
    rebalance of every layer when the peak exceeds MAX_M.
    Drop-in for `for m in layers: m.rebalance()`: call the instance after
    backward.

    device_gate=True (the default): the comparison is made on the device by
    concord_rebalance_group, two launches over a plan of every layer, so a
    call makes no host read and a training step that includes it can be
    captured in one HIP graph; the call returns None and `fires` reads a
    device counter.  Layers with allow_tickdown, or a rebalance statistics
    hook, take the host-gated path.  The plan holds the device addresses of
    each layer's state: after moving or replacing a layer's tensors the next
    call rebuilds it (each eager call compares the addresses).
    device_gate=False: one host read of the peak per call, and the call
    returns True when it fired, as in the reference."""

    def __init__(self, layers, device_gate=True):
        self.layers = [m for m in (layers or []) if hasattr(m, "rebalance")]
        self.MAX_M = max((getattr(m, "MAX_M", 24000) for m in self.layers), default=24000)
        self.device_gate = bool(device_gate)
        self.row_all = None
        self.col_all = None
        self._peak = None
        self._plan = None
        self._plan_sig = None
        self._plan_ws = None
        self._plan_words = 0
        self._fires_dev = None
        self._host_fires = 0
        self.calls = 0

    @property
    def fires(self):
        """Number of calls that fired (reads the device counter: one host
        synchronisation)."""
        dev = 0 if self._fires_dev is None else int(self._fires_dev.item())
        return self._host_fires + dev

    def _wire(self):
        """Repoint the per-layer watermark buffers at slices of the shared
        slabs (once, after the first backward; the slabs start at zero)."""
        dev = self.layers[0].packed_w.device
        rs = [m._row_max_buf.shape[0] for m in self.layers]
        cs = [m._col_max_buf.shape[0] for m in self.layers]
        self.row_all = torch.zeros(sum(rs), dtype=torch.int32, device=dev)
        self.col_all = torch.zeros(sum(cs), dtype=torch.int32, device=dev)
        self._peak = torch.zeros(1, dtype=torch.int32, device=dev)
        self._fires_dev = torch.zeros(1, dtype=torch.int32, device=dev)
        ro = co = 0
        for m, n, k in zip(self.layers, rs, cs):
            m._row_max_buf = self.row_all[ro:ro + n]
            ro += n
            m._col_max_buf = self.col_all[co:co + k]
            co += k
        _stats_workspace(dev, ro + co, 0)

    def peak(self):
        """Device tensor with the largest watermark of every layer (no host read)."""
        ws = _stats_workspace(self.row_all.device, self.row_all.numel() + self.col_all.numel(), 0)
        C.check(C.lib().concord_watermark_peak(
            C.ptr(self.row_all), self.row_all.numel(), C.ptr(self.col_all), self.col_all.numel(),
            C.ptr(self._peak), C.ptr(ws), ws.numel(), C.stream_of(self.row_all.device)), "watermark_peak")
        return self._peak

    def _group_tensors(self, m):
        return (m.packed_w, m.row_exp, m.col_exp, m._row_max_buf, m._col_max_buf, m._row_max_hwm,
                m._col_max_hwm, m._reb_seed)

    def _use_group(self):
        return (self.device_gate and _REB_STATS is None
                and not any(getattr(m, "allow_tickdown", False) for m in self.layers))

    def _ensure_plan(self):
        """Build (or rebuild, when a layer's tensors moved) the device plan of
        concord_rebalance_group."""
        sig = tuple(0 if t is None else t.data_ptr() for m in self.layers for t in self._group_tensors(m))
        if self._plan is not None and sig == self._plan_sig:
            return
        n = len(self.layers)
        rec = (ctypes.c_int64 * (n * C.RG_FIELDS))()
        for i, m in enumerate(self.layers):
            pw, re, ce, rm, cm, rh, chw, seed = self._group_tensors(m)
            N, K = _check_packed(pw, re, ce)
            r = i * C.RG_FIELDS
            rec[r + C.RG_PACKED] = pw.data_ptr()
            rec[r + C.RG_LD] = pw.stride(0)
            rec[r + C.RG_ROW_EXP] = re.data_ptr()
            rec[r + C.RG_COL_EXP] = ce.data_ptr()
            rec[r + C.RG_ROW_MAX] = rm.data_ptr()
            rec[r + C.RG_COL_MAX] = cm.data_ptr()
            rec[r + C.RG_ROW_HWM] = rh.data_ptr() if rh is not None else 0
            rec[r + C.RG_COL_HWM] = chw.data_ptr() if chw is not None else 0
            rec[r + C.RG_SEED] = seed.data_ptr()
            rec[r + C.RG_N] = N
            rec[r + C.RG_K] = K
            rec[r + C.RG_MAX_M] = int(m.MAX_M)
            rec[r + C.RG_EXP_MAX] = int(m.EXP_MAX)
            rec[r + C.RG_EXP_MIN] = int(m.EXP_MIN)
        plen = n * C.RG_FIELDS + 2 * (n + 1)
        plan = (ctypes.c_int64 * plen)()
        words = ctypes.c_int64(0)
        C.check(C.lib().concord_rebalance_group_plan(rec, n, plan, plen, ctypes.byref(words)),
                "rebalance_group_plan")
        dev = self.layers[0].packed_w.device
        self._plan = torch.tensor(list(plan), dtype=torch.int64).to(dev)
        self._plan_words = int(words.value)
        self._plan_ws = torch.empty(self._plan_words, dtype=torch.int32, device=dev)
        self._plan_sig = sig

    def __call__(self):
        if not self.layers:
            return False
        self.calls += 1
        if self.row_all is None:
            if getattr(self.layers[0], "_row_max_buf", None) is None:
                return False
            self._wire()
            return False
        if self._use_group():
            self._ensure_plan()
            peak = self.peak()
            C.check(C.lib().concord_rebalance_group(
                C.ptr(self._plan), len(self.layers), C.ptr(peak), int(self.MAX_M), C.ptr(self._fires_dev),
                C.ptr(self._plan_ws), self._plan_ws.numel() * 4, self._plan_words,
                C.stream_of(peak.device)), "rebalance_group")
            return None
        if int(self.peak().item()) > self.MAX_M:
            for m in self.layers:
                m.rebalance()
            self._host_fires += 1
            return True
        return False


def reference_state_dict(module):
    """module.state_dict() without this build's '_extra_state' entries: the
    key set of the reference classes (their registered buffers and bias,
    concord/packed_b.py:1445-1492), loadable into them with strict=True."""
    return {k: v for k, v in module.state_dict().items()
            if not (k == '_extra_state' or k.endswith('._extra_state'))}


@torch.no_grad()
def consolidated_state_dict(layers, names):
    """Deploy export (notebook/src/concord_winner.py:328-341): each layer's
    consolidated_weight() (s_fast dropped) as name + '.weight', its bias as
    name + '.bias'; conv weights as (out, in, kh, kw); plain bf16
    tensors for safetensors / nn.Linear / nn.Conv2d."""
    out = {}
    for name, m in zip(names, layers):
        W = m.consolidated_weight()
        if isinstance(m, ConcordConv2dPackedB):
            W = W.view(m.out_channels, m.in_channels, m.kh, m.kw)
        out[name + '.weight'] = W
        if getattr(m, 'bias', None) is not None:
            out[name + '.bias'] = m.bias.detach().clone()
    return out
