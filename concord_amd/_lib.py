"""ctypes binding of libconcord_amd.so (the gfx950 kernels behind include/concord_amd.h).

The library is required: there is no fallback.  If it is missing the import of
any compute entry point raises, with the command that builds it.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libconcord_amd.so")

MASS_PRESERVE = 1 << 0
APPLY_CHASE = 1 << 1
TRACK_REBALANCE = 1 << 2
GF_TRUST_REGION = 1 << 3
GF_CONSOLIDATION = 1 << 4
COHPRE = 1 << 5
FIXED_COH = 1 << 6
RATIO_COH = 1 << 7
EMIT_WEIGHT = 1 << 8
PROTO_CONSF = 1 << 9
MUON = 1 << 10
SALT_PREBUMPED = 1 << 16

OK, EINVAL, ELAUNCH, EWORKSPACE = 0, -1, -2, -3

# byte offset of the scratch region in the update-side workspace (after its
# 256-byte counter area); concord_rebalance leaves the row ticks and then the
# column ticks (int32) at its start
WS_SCRATCH = 256

# record layout of concord_rebalance_group_plan's layer table (int64 fields)
RG_FIELDS = 16
(RG_PACKED, RG_LD, RG_ROW_EXP, RG_COL_EXP, RG_ROW_MAX, RG_COL_MAX, RG_ROW_HWM, RG_COL_HWM, RG_SEED,
 RG_N, RG_K, RG_MAX_M, RG_EXP_MAX, RG_EXP_MIN) = range(14)


class UpdateParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in (
        "alpha", "beta1", "weight_decay", "step_cap", "v_scale", "precond_p",
        "gf_consol", "drift_cancel_C", "alpha_v_fast", "wd_sv", "wd_sf",
        "gf_trust_delta_sq", "gate_gain")] + [("mantissa_bias", ctypes.c_int32)]


class DeviceScalars(ctypes.Structure):
    _fields_ = [("lr", ctypes.c_void_p), ("eps", ctypes.c_void_p),
                ("chase_floor", ctypes.c_void_p), ("leak_floor", ctypes.c_void_p),
                ("v_bc", ctypes.c_void_p), ("salt_counter", ctypes.c_void_p),
                ("consolidate", ctypes.c_void_p)]


# (name, restype, argtypes); P = pointer, I = int64, i = int32, F = float, D = double
_P, _I, _i, _F, _D, _Z = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
                          ctypes.c_double, ctypes.c_size_t)
_SIGS = {
    "concord_last_error": (ctypes.c_char_p, []),
    "concord_version": (ctypes.c_int, []),
    "concord_workspace_bytes": (_Z, [_I, _I, _I]),
    "concord_salt_bump": (ctypes.c_int, [_P, _P]),
    "concord_materialize": (ctypes.c_int, [_P, _I, _P, _P, _I, _I, _i, ctypes.c_int, _P, _I, _P]),
    "concord_materialize_gated": (ctypes.c_int, [_P, _I, _P, _P, _I, _I, _i, _F, _P, _I, _P]),
    "concord_apply_adamw": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P,
                                           _I, _I, _I, ctypes.POINTER(UpdateParams),
                                           ctypes.POINTER(DeviceScalars), ctypes.c_uint32, _P]),
    "concord_apply_sgd": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _P, _P, _P, _P, _I, _I, _P, _i,
                                         _F, _F, _F, _P, ctypes.c_uint32, _P]),
    "concord_vhat_ema": (ctypes.c_int, [_P, _I, _I, _I, _D, _P, _P, _P, _P, _P, _P, _P, _Z, _P]),
    "concord_rebalance": (ctypes.c_int, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _i, _i, _i,
                                         ctypes.c_int, ctypes.c_int, _P, _Z, _P]),
    "concord_rebalance_noalloc": (ctypes.c_int, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _I, _I, _i, _i, _i,
                                                 ctypes.c_int, ctypes.c_int, _P]),
    "concord_rebalance_group_plan": (ctypes.c_int, [_P, _i, _P, _I, _P]),
    "concord_rebalance_group": (ctypes.c_int, [_P, _i, _P, _i, _P, _P, _Z, _I, _P]),
    "concord_load_weights": (ctypes.c_int, [_P, _I, _I, _I, _i, _i, _i, ctypes.c_int, _P, _I, _P,
                                            _P, _P]),
    "concord_gemm_workspace_bytes": (_Z, [_I, _I, _I]),
    "concord_dqgemm_fwd": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _i, _P, _P, _I, _I, _I, _I, _P, _Z,
                                          _P]),
    "concord_dqgemm_dgrad": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _i, _P, _I, _I, _I, _I, _P, _Z,
                                            _P]),
    "concord_wgrad": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_wgrad_vhat": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _D, _P, _P, _P, _P, _P,
                                          _P, _P, _P, _Z, _P, _Z, _P]),
    "concord_dgrad_wgrad_vhat": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _i, _P, _I, _P, _I, _P, _I, _I, _I,
                                                 _I, _D, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _P, _Z, _P]),
    "concord_dgrad_wgrad_update": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _I, _P, _I, ctypes.c_int,
                                                   ctypes.c_int, _I, _I, _I, _D, _P, _P, _P, _P, _P, _P, _I, _P,
                                                   ctypes.POINTER(UpdateParams), ctypes.POINTER(DeviceScalars),
                                                   ctypes.c_uint32, _P, _Z, _P, _Z, _P, _P]),
    "concord_wgrad_update_fault": (ctypes.c_int, [_P, _Z, _P, _P]),
    "concord_muon_workspace_bytes": (_Z, [_I, _I]),
    "concord_muon_ns5": (ctypes.c_int, [_P, _I, _I, _I, _F, _P, _I, _P, _Z, _P]),
    "concord_gemm_bf16_fwd": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_gemm_bf16_dgrad": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_gemm_sym_workspace_bytes": (_Z, [_I, _I, ctypes.c_int]),
    "concord_diag_dma_copy": (ctypes.c_int, [_P, _P, _Z, _P]),
    "concord_diag_l2_stream": (ctypes.c_int, [_P, _Z, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P,
                                              _P]),
    "concord_gemm_bf16_sym": (ctypes.c_int, [_P, _I, _P, _I, ctypes.c_int, _P, _I, _I, _I, _P, _Z, _P]),
    "concord_bias_grad": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _Z, _P]),
    "concord_stats_workspace_bytes": (_Z, [_I, _I]),
    "concord_noise_workspace_bytes": (_Z, [_I, _I]),
    "concord_iso_noise": (ctypes.c_int, [_P, _I, _I, _I, _P, _P, _P, _Z, _P]),
    "concord_conv_im2col": (ctypes.c_int, [_P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "concord_conv_col2im": (ctypes.c_int, [_P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P]),
    "concord_conv_col2im_fits": (ctypes.c_int, [_I, _I, _I, _I]),
    "concord_conv_implicit_ok": (ctypes.c_int, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "concord_conv_workspace_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I]),
    "concord_conv_weight_taps": (ctypes.c_int, [_P, _I, _P, _P, _I, _I, _I, _i, _F, _P, _P]),
    "concord_conv_grad_from_taps": (ctypes.c_int, [_P, _I, _I, _I, _P, _I, _P]),
    "concord_conv_fwd": (ctypes.c_int, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_conv_dgrad": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_conv_wgrad": (ctypes.c_int, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _Z, _P]),
    "concord_conv_wgrad_vhat": (ctypes.c_int, [_P, _P, _P, _P, _I] + [_I] * 11 +
                                [_D, _P, _P, _P, _P, _P, _P, _P, _P, _Z, _P, _Z, _P]),
    "concord_sigmag_noise_workspace_bytes": (_Z, [_I, _I, _I]),
    "concord_sigmag_noise": (ctypes.c_int, [_P, _I, _P, _I, _P, _I, _I, _I, _I, _P, _P, _P, _Z, _P]),
    "concord_watermark_peak": (ctypes.c_int, [_P, _I, _P, _I, _P, _P, _Z, _P]),
    "concord_coherence_sum": (ctypes.c_int, [_P, _I, _I, _I, _F, _P, _P, _Z, _P]),
}

_lib = None


class ConcordError(RuntimeError):
    pass


def lib():
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ConcordError(
                f"concord_amd: {LIB_PATH} is missing; build it with "
                "`python -m concord_amd.build` (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return list(_SIGS)


def check(rc, what):
    if rc != OK:
        msg = lib().concord_last_error().decode(errors="replace")
        if rc == EINVAL:
            raise ValueError(f"{what}: {msg}")
        raise ConcordError(f"{what} failed ({rc}): {msg}")


def ptr(t):
    """Device address of a tensor (None -> NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def stream_of(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_device_tensor(t, name):
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise RuntimeError(
            f"concord_amd: {name} must be a ROCm device tensor (got "
            f"{getattr(t, 'device', type(t))}); the packed path has no CPU implementation")
