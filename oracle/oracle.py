"""ctypes front end of the CPU oracle (oracle/concord_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product package (concord_amd) never imports it.

Arrays are numpy; the functions mutate their in/out arguments in place like the
reference kernels do (concord/packed_b.py:422-703, 959-1095).
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libconcord_oracle.so")

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


class UpdateParams(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in (
        "alpha", "beta1", "weight_decay", "step_cap", "v_scale", "precond_p",
        "gf_consol", "drift_cancel_C", "alpha_v_fast", "wd_sv", "wd_sf",
        "gf_trust_delta_sq", "gate_gain")] + [("mantissa_bias", ctypes.c_int32)]


class UpdateScalars(ctypes.Structure):
    _fields_ = [(n, ctypes.c_float) for n in (
        "lr", "eps", "chase_floor", "leak_floor", "v_bc")] + [
        ("salt", ctypes.c_int32), ("consolidate", ctypes.c_int32)]


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i64, i32, f32, f64, u32 = (ctypes.c_int64, ctypes.c_int32, ctypes.c_float,
                                   ctypes.c_double, ctypes.c_uint32)
        L.oracle_hash_uniform.restype = f32
        L.oracle_hash_uniform.argtypes = [i32, i32, i32]
        L.oracle_philox4x32_10.argtypes = [P, P]
        L.oracle_tl_rand.restype = f32
        L.oracle_tl_rand.argtypes = [i32, i32]
        L.oracle_f2i.restype = i32
        L.oracle_f2i.argtypes = [f32]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f32_to_bf16.argtypes = [f32]
        L.oracle_pow_p.restype = f32
        L.oracle_pow_p.argtypes = [f32, f32]
        L.oracle_drift_cancel_C.restype = f64
        L.oracle_drift_cancel_C.argtypes = [f64, f64, f64, ctypes.c_int, ctypes.c_int]
        L.oracle_materialize.argtypes = [P, P, P, i64, i64, i32, ctypes.c_int, P]
        L.oracle_materialize_gated.argtypes = [P, P, P, i64, i64, i32, f32, P]
        L.oracle_apply_adamw.argtypes = [P, P, P, P, P, P, P, P, P, f32, P, i64, i64,
                                         ctypes.POINTER(UpdateParams),
                                         ctypes.POINTER(UpdateScalars), u32]
        L.oracle_apply_sgd.argtypes = [P, P, P, P, P, P, P, i64, i64, f32, i32, f32,
                                       f32, f32, i32, u32]
        L.oracle_i8_medians.argtypes = [P, i64, i64, P, P]
        L.oracle_frob_sumsq.restype = f32
        L.oracle_frob_sumsq.argtypes = [P, i64, i64]
        L.oracle_coherence_sum.restype = f32
        L.oracle_coherence_sum.argtypes = [P, i64, i64, f32]
        L.oracle_iso_draw.restype = f32
        L.oracle_iso_draw.argtypes = [i32, i64]
        L.oracle_iso_noise.argtypes = [P, i64, i64, f32, i32]
        L.oracle_normal_draw_tag.restype = f32
        L.oracle_normal_draw_tag.argtypes = [i32, ctypes.c_uint32, ctypes.c_uint32]
        L.oracle_token_sum.restype = f32
        L.oracle_token_sum.argtypes = [i32, i64]
        L.oracle_sigmag_combine.argtypes = [P, P, i64, i64, f32, f32, f32]
        L.oracle_muon_ns5.argtypes = [P, i64, i64, f32, P]
        L.oracle_rebalance.argtypes = [P, P, P, P, P, P, P, i64, i64, i32, i32, i32,
                                       i32, ctypes.c_int]
        L.oracle_vhat_ema.argtypes = [P, i64, i64, P, P, P, f64]
        L.oracle_load_weights.argtypes = [P, i64, i64, i32, i32, i32, ctypes.c_int,
                                          P, P, P]
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def set_threads(n):
    lib().oracle_set_threads(int(n))


def hash_uniform(x, pos, salt):
    return lib().oracle_hash_uniform(int(np.int32(x)), int(np.int32(pos)), int(np.int32(salt)))


def philox4x32_10(ctr, key):
    c = np.asarray(ctr, dtype=np.uint32).copy()
    k = np.asarray(key, dtype=np.uint32).copy()
    lib().oracle_philox4x32_10(_p(c), _p(k))
    return c


def tl_rand(seed, offset):
    return lib().oracle_tl_rand(int(np.int32(seed)), int(np.int32(offset)))


def f32_to_bf16_bits(x):
    return lib().oracle_f32_to_bf16(float(np.float32(x)))


def pow_p(x, p):
    return lib().oracle_pow_p(float(np.float32(x)), float(np.float32(p)))


def drift_cancel_C(alpha, alpha_v_fast, alpha_v_slow=0.0, refit_period=1,
                   mass_preserve=True):
    return lib().oracle_drift_cancel_C(alpha, alpha_v_fast, alpha_v_slow,
                                       int(refit_period), int(bool(mass_preserve)))


def materialize(packed, row_exp, col_exp, mantissa_bias=15, consolidated=False):
    N, K = packed.shape
    out = np.empty((N, K), dtype=np.uint16)
    lib().oracle_materialize(_p(packed), _p(row_exp), _p(col_exp), N, K,
                             int(mantissa_bias), int(bool(consolidated)), _p(out))
    return out


def materialize_gated(packed, row_exp, col_exp, fast_gain, mantissa_bias=15):
    N, K = packed.shape
    out = np.empty((N, K), dtype=np.uint16)
    lib().oracle_materialize_gated(_p(np.ascontiguousarray(packed, dtype=np.int32)), _p(row_exp),
                                   _p(col_exp), N, K, int(mantissa_bias), float(fast_gain), _p(out))
    return out


def apply_adamw(packed, grad_bf16, weight_bf16, row_exp, col_exp, row_max, col_max,
                v_row, v_col, sum_v_inv, coh_pre, params, scalars, flags):
    """In place on packed / weight_bf16 / row_max / col_max / coh_pre."""
    N, K = packed.shape
    dummy_f = np.zeros(1, np.float32)
    lib().oracle_apply_adamw(
        _p(packed), _p(grad_bf16), _p(weight_bf16 if weight_bf16 is not None else np.zeros(1, np.uint16)),
        _p(row_exp), _p(col_exp), _p(row_max), _p(col_max),
        _p(v_row if v_row is not None else dummy_f), _p(v_col if v_col is not None else dummy_f),
        float(sum_v_inv), _p(coh_pre if coh_pre is not None else dummy_f), N, K,
        ctypes.byref(params), ctypes.byref(scalars), int(flags))


def apply_sgd(packed, grad_bf16, weight_bf16, row_exp, col_exp, row_max, col_max,
              lr, mantissa_bias, alpha, beta1, alpha_v_fast, salt, flags):
    N, K = packed.shape
    lib().oracle_apply_sgd(_p(packed), _p(grad_bf16),
                           _p(weight_bf16 if weight_bf16 is not None else np.zeros(1, np.uint16)),
                           _p(row_exp), _p(col_exp), _p(row_max), _p(col_max), N, K,
                           float(lr), int(mantissa_bias), float(alpha), float(beta1),
                           float(alpha_v_fast), int(np.int32(salt)), int(flags))


def i8_medians(packed):
    N, K = packed.shape
    rm = np.zeros(N, np.int32)
    cm = np.zeros(K, np.int32)
    lib().oracle_i8_medians(_p(packed), N, K, _p(rm), _p(cm))
    return rm, cm


def rebalance(packed, row_exp, col_exp, row_max, col_max, row_med=None, col_med=None,
              max_m=24000, exp_max=7, exp_min=-8, seed=0, allow_tickdown=False):
    """In place on packed / row_exp / col_exp."""
    N, K = packed.shape
    if row_med is None or col_med is None:
        row_med, col_med = i8_medians(packed)
    lib().oracle_rebalance(_p(packed), _p(row_exp), _p(col_exp), _p(row_max), _p(col_max),
                           _p(row_med), _p(col_med), N, K, int(max_m), int(exp_max),
                           int(exp_min), int(np.int32(seed)), int(bool(allow_tickdown)))


def vhat_ema(grad_bf16, v_row, v_col, beta2=0.999):
    """In place on v_row / v_col; returns sum_v_inv (float32)."""
    N, K = grad_bf16.shape
    s = np.zeros(1, np.float32)
    lib().oracle_vhat_ema(_p(grad_bf16), N, K, _p(v_row), _p(v_col), _p(s), float(beta2))
    return s[0]


def frob_sumsq(grad_bf16):
    g = np.ascontiguousarray(grad_bf16, dtype=np.uint16)
    return np.float32(lib().oracle_frob_sumsq(_p(g), g.shape[0], g.shape[1]))


def coherence_sum(packed, drift_cancel_C):
    """Sum of the gate's Wiener gain over the words (fixed library order)."""
    p = np.ascontiguousarray(packed, dtype=np.int32)
    return np.float32(lib().oracle_coherence_sum(_p(p), p.shape[0], p.shape[1], float(drift_cancel_C)))


def iso_draws(seed, n, start=0):
    """Draws start .. start + n - 1 of the isotropic noise stream `seed`
    (element e: draw e & 3 of Philox block e >> 2)."""
    f = lib().oracle_iso_draw
    return np.array([f(int(seed), start + i) for i in range(n)], dtype=np.float32)


TAG_ISO = 0x6E6F6973


def normal_draw_tag(seed, idx, tag):
    """One Box-Muller draw (cos output) on Philox block idx under key (seed, tag)."""
    return np.float32(lib().oracle_normal_draw_tag(int(seed), int(idx) & 0xFFFFFFFF, int(tag)))


TAG_TOKEN = 0x5369676D


def token_draws(seed, M):
    """The per-token draws eps_0 .. eps_{M-1} of the Sigma_g noise."""
    f = lib().oracle_normal_draw_tag
    return np.array([f(int(seed), m, TAG_TOKEN) for m in range(M)], dtype=np.float32)


def token_sum(seed, M):
    return np.float32(lib().oracle_token_sum(int(seed), int(M)))


def sigmag_combine(grad_bf16, P_bf16, S, M, sigma):
    g = np.ascontiguousarray(grad_bf16, dtype=np.uint16).copy()
    P = np.ascontiguousarray(P_bf16, dtype=np.uint16)
    lib().oracle_sigmag_combine(_p(g), _p(P), g.shape[0], g.shape[1], float(S), float(max(M, 1)),
                                float(sigma))
    return g


def iso_noise(grad_bf16, sigma, salt):
    """Isotropic noise injection on bf16 bits (returns a new array)."""
    g = np.ascontiguousarray(grad_bf16, dtype=np.uint16).copy()
    lib().oracle_iso_noise(_p(g), g.shape[0], g.shape[1], float(sigma), int(salt))
    return g


def muon_ns5(grad_bf16, gamma=None):
    """O = bf16(gamma * NS5(g / ||g||)) as bf16 bits (gamma = sqrt(max(N, K)))."""
    g = np.ascontiguousarray(grad_bf16, dtype=np.uint16)
    N, K = g.shape
    if gamma is None:
        gamma = float(np.float32(np.sqrt(np.float32(max(N, K)))))
    out = np.zeros((N, K), np.uint16)
    lib().oracle_muon_ns5(_p(g), N, K, float(gamma), _p(out))
    return out


def load_weights(W, exp_min=-8, exp_max=7, mantissa_bias=15, finetune=False):
    W = np.ascontiguousarray(W, dtype=np.float32)
    N, K = W.shape
    packed = np.zeros((N, K), np.int32)
    re = np.zeros(N, np.int8)
    ce = np.zeros(K, np.int8)
    lib().oracle_load_weights(_p(W), N, K, int(exp_min), int(exp_max),
                              int(mantissa_bias), int(bool(finetune)),
                              _p(packed), _p(re), _p(ce))
    return packed, re, ce


def bf16_bits_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits_array(x):
    """Vectorised RNE fp32 -> bf16 bits (NaN -> 0x7FC0), same rule as the C oracle."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FC0
    return r


def unpack(packed):
    p = packed.astype(np.int32)
    sf = p >> 16
    ss = (p << 16) >> 24
    vs = (p << 24) >> 24
    return sf, ss, vs


def pack(sf, ss, vs):
    sf = np.asarray(sf, np.int64)
    ss = np.asarray(ss, np.int64)
    vs = np.asarray(vs, np.int64)
    u = ((sf & 0xFFFF) << 16) | ((ss & 0xFF) << 8) | (vs & 0xFF)
    return u.astype(np.uint32).view(np.int32)
