"""Pin the CPU oracle by what the mathematics fixes: published known answers,
closed forms, conservation laws, special cases and expectations.

Complements tests/test_oracle_golden.py (the reference's own outputs).  Each
check is chosen so that a plausible slip in the oracle (a dropped term, a
swapped operand, a wrong shift kind or stream salt) fails it.
"""
import math

import numpy as np
import pytest
import torch

# ---------------------------------------------------------------- RNG pieces


def test_philox_known_answers(oracle):
    """Random123 kat_vectors for philox4x32-10 (Salmon et al., SC'11)."""
    kat = [
        ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
        ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
        ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
         [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    ]
    for ctr, key, want in kat:
        assert list(oracle.philox4x32_10(ctr, key)) == want


def test_tl_rand_mapping(oracle):
    # seed 0, offset 0 -> counter (0,0,0,0) key (0,0): word 0 is the first KAT word
    w = 0x6627E8D5
    assert oracle.tl_rand(0, 0) == np.float32(w) * np.float32(4.6566127342e-10)
    # a negative seed sign-extends into the high key word
    c = oracle.philox4x32_10([7, 0, 0, 0], [0xFFFFFFFE, 0xFFFFFFFF])[0]
    x = np.int32(np.uint32(c).view(np.int32))
    x = -x - 1 if x < 0 else x
    assert oracle.tl_rand(-2, 7) == np.float32(x) * np.float32(4.6566127342e-10)
    u = np.array([oracle.tl_rand(3, i) for i in range(20000)])
    assert u.min() >= 0 and u.max() < 1
    assert abs(u.mean() - 0.5) < 0.01 and abs(u.var() - 1 / 12) < 0.005


def test_hash_uses_arithmetic_shifts(oracle):
    # hand-evaluated: x = INT32_MIN, pos = salt = 0 -> h = 0x7F07CF80 with
    # arithmetic >>; logical >> would give 0x81084840.
    assert oracle.hash_uniform(-(2 ** 31), 0, 0) == np.float32(0x07CF80) / np.float32(2 ** 24)
    assert oracle.hash_uniform(0, 0, 0) == 0.0
    # x ^ salt ^ pos enters symmetrically
    assert oracle.hash_uniform(5, 9, 3) == oracle.hash_uniform(3, 9, 5) == oracle.hash_uniform(9, 5, 3)


def test_hash_uniformity(oracle):
    rng = np.random.default_rng(0)
    xs = rng.integers(-30000, 30000, 20000)
    u = np.array([oracle.hash_uniform(int(x), (i << 16) ^ 77, 12345) for i, x in enumerate(xs)])
    assert u.min() >= 0 and u.max() < 1
    assert np.all(u * 2 ** 24 == np.floor(u * 2 ** 24))
    assert abs(u.mean() - 0.5) < 0.01
    h, _ = np.histogram(u, bins=16, range=(0, 1))
    assert h.min() > 0.85 * len(u) / 16


# ------------------------------------------------------------ scalar helpers


def test_drift_cancel_constants(oracle):
    # concord/packed_b.py:69-70 and the mass-preserve formula at 100-101
    assert abs(oracle.drift_cancel_C(0.1, 0.001) - 0.018036072) < 1e-8
    assert abs(oracle.drift_cancel_C(0.1, 0.001, mass_preserve=False) - 0.0090817) < 1e-6
    # periodic leak raises rho: alpha_v_slow/T_r = 0.00125 -> C ~ 0.0204 (legacy)
    assert abs(oracle.drift_cancel_C(0.1, 0.001, 0.0025, 2, mass_preserve=False) - 0.0204) < 5e-4


def test_pow_p(oracle):
    for x in [1e-30, 3e-12, 0.25, 1.0, 7.5, 1e20]:
        assert oracle.pow_p(x, 0.5) == np.sqrt(np.float32(x))
        assert oracle.pow_p(x, 0.0) == 1.0
        for p in [0.25, 0.4, 1.0]:
            want = float(np.float32(x)) ** float(np.float32(p))
            assert abs(oracle.pow_p(x, p) - want) <= 4e-6 * want


def test_bf16_rounding_matches_torch(oracle):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(10000) * 10.0 ** rng.uniform(-30, 30, 10000)).astype(np.float32)
    x[:4] = [0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8]   # exact ties
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits_array(x), want)
    assert all(oracle.f32_to_bf16_bits(v) == w for v, w in zip(x[:200], want[:200]))


def test_f2i_policy(oracle):
    assert oracle.lib().oracle_f2i(float("nan")) == 0
    assert oracle.lib().oracle_f2i(3e9) == 2 ** 31 - 1
    assert oracle.lib().oracle_f2i(-3e9) == -(2 ** 31)
    assert oracle.lib().oracle_f2i(-2.7) == -2


# ------------------------------------------------------------ decode family


def _rand_state(rng, N, K, sf=(-30000, 30000)):
    sfv = rng.integers(sf[0], sf[1], (N, K))
    ss = rng.integers(-128, 128, (N, K))
    vs = rng.integers(-128, 128, (N, K))
    return sfv, ss, vs


def test_materialize_closed_form(oracle):
    rng = np.random.default_rng(2)
    N, K = 37, 93
    sf, ss, vs = _rand_state(rng, N, K)
    packed = oracle.pack(sf, ss, vs)
    re = rng.integers(-8, 8, N).astype(np.int8)
    ce = rng.integers(-8, 8, K).astype(np.int8)
    for cons in (False, True):
        m = 128 * ss + 128 * vs + (0 if cons else sf)
        exact = m.astype(np.float64) * np.exp2(re[:, None].astype(np.float64) + ce[None, :] - 15)
        want = torch.from_numpy(exact).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        got = oracle.materialize(packed, re, ce, consolidated=cons)
        np.testing.assert_array_equal(got, want)


def test_pack_roundtrip(oracle):
    rng = np.random.default_rng(3)
    sf, ss, vs = _rand_state(rng, 50, 60, sf=(-32768, 32768))
    p = oracle.pack(sf, ss, vs)
    a, b, c = oracle.unpack(p)
    np.testing.assert_array_equal(a, sf)
    np.testing.assert_array_equal(b, ss)
    np.testing.assert_array_equal(c, vs)


def test_i8_medians(oracle):
    rng = np.random.default_rng(4)
    for N, K in [(7, 10), (16, 33), (1, 5)]:
        sf, ss, vs = _rand_state(rng, N, K)
        p = oracle.pack(sf, ss, vs)
        a = np.maximum(np.abs(ss), np.abs(vs))
        rm, cm = oracle.i8_medians(p)
        np.testing.assert_array_equal(rm, np.sort(a, 1)[:, (K - 1) // 2])
        np.testing.assert_array_equal(cm, np.sort(a, 0)[(N - 1) // 2, :])


# --------------------------------------------------------------- update law

def _params(O, **kw):
    d = dict(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0, precond_p=0.5,
             gf_consol=0.0, drift_cancel_C=0.018036072144288578, alpha_v_fast=0.001, wd_sv=0.0,
             wd_sf=0.0, gf_trust_delta_sq=1.0, gate_gain=1.0, mantissa_bias=15)
    d.update(kw)
    return O.UpdateParams(**d)


def _scalars(O, **kw):
    d = dict(lr=5e-4, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0, salt=1,
             consolidate=1)
    d.update(kw)
    return O.UpdateScalars(**d)


def _apply(O, packed, grad_bits, re, ce, P, S, flags, v_row=None, v_col=None, svi=1.0, cp=None):
    N, K = packed.shape
    pk = packed.copy()
    w = np.zeros((N, K), np.uint16)
    rm = np.zeros(N, np.int32)
    cm = np.zeros(K, np.int32)
    vr = v_row if v_row is not None else np.full(N, 1e-4, np.float32)
    vc = v_col if v_col is not None else np.full(K, 1e-4, np.float32)
    O.apply_adamw(pk, grad_bits, w, re, ce, rm, cm, vr, vc, svi, cp, P, S, flags)
    return pk, w, rm, cm


def _mid_state(O, rng, N, K):
    sf = rng.integers(-2000, 2000, (N, K))
    ss = rng.integers(-60, 60, (N, K))
    vs = rng.integers(-60, 60, (N, K))
    return O.pack(sf, ss, vs), np.zeros(N, np.int8), np.zeros(K, np.int8)


def test_chase_conserves_live_mantissa(oracle):
    O = oracle
    rng = np.random.default_rng(5)
    packed, re, ce = _mid_state(O, rng, 30, 40)
    g = np.zeros((30, 40), np.uint16)
    P = _params(O, alpha=0.37, alpha_v_fast=0.0)
    fl = O.APPLY_CHASE | O.MASS_PRESERVE | O.GF_TRUST_REGION
    out, *_ = _apply(O, packed, g, re, ce, P, _scalars(O, lr=0.0), fl)
    sf0, ss0, vs0 = O.unpack(packed)
    sf1, ss1, vs1 = O.unpack(out)
    np.testing.assert_array_equal(sf1 + 128 * ss1 + 128 * vs1, sf0 + 128 * ss0 + 128 * vs0)
    assert (ss1 != ss0).any()
    np.testing.assert_array_equal(vs1, vs0)


def test_mass_preserving_leak_conserves_position(oracle):
    O = oracle
    rng = np.random.default_rng(6)
    packed, re, ce = _mid_state(O, rng, 30, 40)
    g = np.zeros((30, 40), np.uint16)
    P = _params(O, alpha=0.0, alpha_v_fast=0.3)
    fl = O.APPLY_CHASE | O.MASS_PRESERVE
    out, *_ = _apply(O, packed, g, re, ce, P, _scalars(O, lr=0.0), fl)
    sf0, ss0, vs0 = O.unpack(packed)
    sf1, ss1, vs1 = O.unpack(out)
    np.testing.assert_array_equal(ss1 + vs1, ss0 + vs0)
    np.testing.assert_array_equal(sf1, sf0)
    assert (vs1 != vs0).any()
    # without mass preservation the position moves by the leak
    out2, *_ = _apply(O, packed, g, re, ce, P, _scalars(O, lr=0.0), O.APPLY_CHASE)
    _, ss2, vs2 = O.unpack(out2)
    np.testing.assert_array_equal(ss2, ss0)
    assert (vs2 != vs0).any()


def test_consolidate_zero_is_tick_only(oracle):
    O = oracle
    rng = np.random.default_rng(7)
    packed, re, ce = _mid_state(O, rng, 20, 70)
    g = O.f32_to_bf16_bits_array(rng.standard_normal((20, 70)).astype(np.float32) * 1e-3)
    P = _params(O, gf_consol=50.0, beta1=0.2, wd_sv=0.1, wd_sf=0.1)
    fl = (O.APPLY_CHASE | O.MASS_PRESERVE | O.TRACK_REBALANCE | O.GF_TRUST_REGION
          | O.GF_CONSOLIDATION | O.RATIO_COH | O.FIXED_COH | O.EMIT_WEIGHT | O.PROTO_CONSF)
    out, w, rm, cm = _apply(O, packed, g, re, ce, P, _scalars(O, consolidate=0), fl)
    sf0, ss0, vs0 = O.unpack(packed)
    sf1, ss1, vs1 = O.unpack(out)
    np.testing.assert_array_equal(ss1, ss0)
    np.testing.assert_array_equal(vs1, vs0)
    assert (sf1 != sf0).any()
    assert not w.any() and not rm.any() and not cm.any()


def test_zero_lr_no_chase_is_identity(oracle):
    O = oracle
    rng = np.random.default_rng(8)
    packed, re, ce = _mid_state(O, rng, 20, 30)
    g = O.f32_to_bf16_bits_array(rng.standard_normal((20, 30)).astype(np.float32))
    out, *_ = _apply(O, packed, g, re, ce, _params(O), _scalars(O, lr=0.0),
                     O.GF_TRUST_REGION | O.FIXED_COH | O.COHPRE, cp=np.ones((20, 30), np.float32))
    np.testing.assert_array_equal(out, packed)


def test_zero_state_zero_grad_stays_zero(oracle):
    O = oracle
    z = np.zeros((9, 13), np.int32)
    for fl in [0x7F, 0xFF | O.PROTO_CONSF, O.APPLY_CHASE | O.MASS_PRESERVE | O.GF_CONSOLIDATION]:
        out, *_ = _apply(O, z, np.zeros((9, 13), np.uint16), np.zeros(9, np.int8),
                         np.zeros(13, np.int8), _params(O, gf_consol=5.0), _scalars(O), fl,
                         cp=np.ones((9, 13), np.float32))
        assert not out.any()


def _salt_mean(O, packed, g, re, ce, P, fl, v_row, v_col, svi, T=3000, **sc):
    N, K = packed.shape
    acc = np.zeros((3, N, K))
    acc2 = np.zeros((3, N, K))
    # uniformly random 32-bit salts: the xorshift map is a bijection, so the
    # draw is exactly uniform over salts (structured salts are not)
    salts = np.random.default_rng(99).integers(-2 ** 31, 2 ** 31, T)
    for s in range(T):
        out, *_ = _apply(O, packed, g, re, ce, P, _scalars(O, salt=int(salts[s]), **sc),
                         fl, v_row, v_col, svi)
        f = np.stack(O.unpack(out)).astype(np.float64)
        acc += f
        acc2 += f * f
    mean = acc / T
    sem = np.sqrt(np.maximum(acc2 / T - mean ** 2, 1.0 / T) / T)
    return mean, sem


def test_update_expectation_matches_real_valued_rule(oracle):
    """E over SR salts of each stage of the integer update == the real-valued
    rule of experiments/cpu_dynamics/concord_ref.py:108-156 (ratio gates +
    evaporation), in mantissa units (u = s_fast, S = 128 s_slow, A = 128 v_slow).

    Stages are checked one at a time: the reference's SR hash is an xorshift,
    linear over GF(2), so within one update the chase draw equals the tick draw
    XOR a constant fixed by the element; a chained stage is only unbiased when
    the earlier stage is deterministic."""
    O = oracle
    rng = np.random.default_rng(9)
    N, K = 8, 16
    sf0 = rng.integers(-1500, 1500, (N, K))
    ss0 = rng.integers(-50, 50, (N, K))
    vs0 = rng.integers(-50, 50, (N, K))
    packed = O.pack(sf0, ss0, vs0)
    re = np.full(N, 2, np.int8)
    ce = np.zeros(K, np.int8)
    gf = (rng.standard_normal((N, K)) * 3e-4).astype(np.float32)
    g = O.f32_to_bf16_bits_array(gf)
    v_row = np.full(N, 2e-6, np.float32)
    v_col = np.full(K, 2e-6, np.float32)
    svi = np.float32(1.0 / (N * 2e-6))
    lr, kappa, cf, lf, alpha, av, C = 2e-3, 30.0, 0.6, 0.4, 0.1, 0.05, 0.018036072144288578
    base = O.MASS_PRESERVE | O.GF_TRUST_REGION | O.GF_CONSOLIDATION | O.RATIO_COH | O.FIXED_COH
    u, S, A = sf0.astype(np.float64), 128.0 * ss0, 128.0 * vs0
    vhat = v_row[:, None].astype(np.float64) * v_col[None, :] * svi
    mu = C * (S - A)
    nse = u - mu
    coh = mu * mu / (mu * mu + nse * nse + 1e-30)
    gq = O.bf16_bits_to_f32(g).astype(np.float64)     # the update consumes bf16(grad)
    step = np.clip(gq / np.sqrt(vhat + 1e-10), -10, 10)
    sc = dict(chase_floor=cf, leak_floor=lf)

    # 1. drive + evaporation (no chase)
    P = _params(O, alpha=alpha, alpha_v_fast=av, gf_consol=kappa, drift_cancel_C=C)
    mean, sem = _salt_mean(O, packed, g, re, ce, P, base, v_row, v_col, svi, lr=lr, **sc)
    want = u - lr * step * 2.0 ** 13 - lr * kappa * (1 - coh) * u
    assert (np.abs(mean[0] - want) / sem[0]).max() < 6.0
    np.testing.assert_array_equal(mean[1:], np.stack([ss0, vs0]))

    # 2. chase alone (lr = 0: the tick is deterministic zero)
    P = _params(O, alpha=alpha, alpha_v_fast=0.0, gf_consol=kappa, drift_cancel_C=C)
    mean, sem = _salt_mean(O, packed, g, re, ce, P, base | O.APPLY_CHASE, v_row, v_col, svi,
                           lr=0.0, **sc)
    tr = alpha * (cf + (1 - cf) * coh) * u
    assert (np.abs(mean[1] - (S + tr) / 128) / sem[1]).max() < 6.0
    assert (np.abs(mean[0] - (u - tr)) / sem[0]).max() < 6.0

    # 3. leak alone (alpha = 0: the chase is deterministic zero)
    P = _params(O, alpha=0.0, alpha_v_fast=av, gf_consol=kappa, drift_cancel_C=C)
    mean, sem = _salt_mean(O, packed, g, re, ce, P, base | O.APPLY_CHASE, v_row, v_col, svi,
                           lr=0.0, **sc)
    lk = av * (lf + (1 - lf) * coh) * (S - A)
    assert (np.abs(mean[2] - (A + lk) / 128) / sem[2]).max() < 6.0
    assert (np.abs(mean[1] - (S - lk) / 128) / sem[1]).max() < 6.0


def test_muon_update_expectation_matches_real_valued_rule(oracle):
    """CONCORD_MUON: E over SR salts of the integer update == the tick of
    MuonConcord.step (experiments/cpu_dynamics/exp9_muon.py:58-100), in
    mantissa units, with the drive supplied as its step_:
        u <- u - lr O 2^-(row_exp + col_exp - 15) - lr kappa (1 - coh) u.
    No denominator and no clip (drive entries up to 40 pass whole: a clip
    at the v-hat arm's 10, or a division by sqrt(v-hat + eps), fails), and
    v-hat is never read (NaN v_row / v_col / sum_v_inv change nothing).
    The chase and the leak downstream are the v-hat arm's, pinned above."""
    O = oracle
    rng = np.random.default_rng(19)
    N, K = 8, 16
    sf0 = rng.integers(-1500, 1500, (N, K))
    ss0 = rng.integers(-50, 50, (N, K))
    vs0 = rng.integers(-50, 50, (N, K))
    packed = O.pack(sf0, ss0, vs0)
    re = np.full(N, 2, np.int8)
    ce = np.zeros(K, np.int8)
    drive = np.clip(rng.standard_normal((N, K)) * 15.0, -40.0, 40.0).astype(np.float32)
    drive[0, :4] = [40.0, -40.0, 25.0, -12.5]
    d = O.f32_to_bf16_bits_array(drive)
    v_row = np.full(N, 2e-6, np.float32)
    v_col = np.full(K, 2e-6, np.float32)
    svi = np.float32(1.0 / (N * 2e-6))
    lr, kappa, C = 1e-4, 30.0, 0.018036072144288578
    base = (O.MASS_PRESERVE | O.GF_TRUST_REGION | O.GF_CONSOLIDATION | O.RATIO_COH | O.FIXED_COH
            | O.MUON)
    u, S, A = sf0.astype(np.float64), 128.0 * ss0, 128.0 * vs0
    mu = C * (S - A)
    nse = u - mu
    coh = mu * mu / (mu * mu + nse * nse + 1e-30)
    Od = O.bf16_bits_to_f32(d).astype(np.float64)      # the update consumes bf16(O)
    P = _params(O, alpha=0.1, alpha_v_fast=0.05, gf_consol=kappa, drift_cancel_C=C)
    sc = dict(chase_floor=0.6, leak_floor=0.4)
    mean, sem = _salt_mean(O, packed, d, re, ce, P, base, v_row, v_col, svi, lr=lr, **sc)
    want = u - lr * Od * 2.0 ** 13 - lr * kappa * (1 - coh) * u
    assert (np.abs(mean[0] - want) / sem[0]).max() < 6.0
    np.testing.assert_array_equal(mean[1:], np.stack([ss0, vs0]))
    # the clipped and the preconditioned drives are far outside that band
    for wrong in (u - lr * np.clip(Od, -10, 10) * 2.0 ** 13 - lr * kappa * (1 - coh) * u,
                  u - lr * Od / np.sqrt(v_row[0] * v_col[0] * svi + 1e-10) * 2.0 ** 13):
        assert (np.abs(mean[0] - wrong) / sem[0]).max() > 50.0
    nan = np.full(N, np.nan, np.float32), np.full(K, np.nan, np.float32)
    flags = base | O.APPLY_CHASE | O.TRACK_REBALANCE
    a = _apply(O, packed, d, re, ce, P, _scalars(O, lr=lr, salt=5, **sc), flags, v_row, v_col, svi)
    b = _apply(O, packed, d, re, ce, P, _scalars(O, lr=lr, salt=5, **sc), flags, nan[0], nan[1],
               float("nan"))
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


def test_sr_streams_are_xor_linked(oracle):
    """The property behind the stage-wise test above, shown directly:
    hash(x, pos, s) XOR hash(y, pos, s ^ c) is independent of the salt s."""
    O = oracle
    pos = (5 << 16) ^ 9
    xs = {int(O.hash_uniform(846, pos, s) * 2 ** 24) ^ int(O.hash_uniform(799, pos, s ^ 0x5A5A5A5A) * 2 ** 24)
          for s in range(1, 5000, 37)}
    assert len(xs) == 1


# -------------------------------------------------------------- rebalance


def _rebal(O, sf, ss, vs, r0, c0, tickdown, seed=1):
    packed = O.pack(sf, ss, vs)
    N, K = packed.shape
    re = np.full(N, r0, np.int8)
    ce = np.full(K, c0, np.int8)
    m = ss * 128 + sf + vs * 128
    rmax = np.abs(m).max(1).astype(np.int32)
    cmax = np.abs(m).max(0).astype(np.int32)
    w0 = m * np.exp2(r0 + c0 - 15.0)
    pk = packed.copy()
    O.rebalance(pk, re, ce, rmax, cmax, seed=seed, allow_tickdown=tickdown)
    sf1, ss1, vs1 = O.unpack(pk)
    w1 = (ss1 * 128 + sf1 + vs1 * 128) * np.exp2(re[:, None].astype(float) + ce[None, :] - 15)
    return w0, w1, ss1, vs1, re, ce


def test_rebalance_invariants(oracle):
    """notebook/src/test_tickdown.py:58-81: value preservation, int8 range,
    deadband, EXP_MIN floor."""
    O = oracle
    rng = np.random.default_rng(10)
    N = K = 64
    ri = lambda lo, hi: rng.integers(lo, hi, (N, K))  # noqa: E731
    # tick-down: exact
    w0, w1, ss, vs, re, ce = _rebal(O, ri(-20, 20), ri(-14, 15), ri(-14, 15), 5, 5, True)
    assert np.abs(w1 - w0).max() == 0 and (re == 4).all() and (ce == 4).all()
    assert np.abs(ss).max() <= 127 and np.abs(vs).max() <= 127
    # tick-up: within SR, exponent +1 on both -> net +2
    w0, w1, ss, vs, re, ce = _rebal(O, ri(-50, 50), np.full((N, K), 100), np.full((N, K), 100), 0, 0, True)
    assert (re == 1).all() and (ce == 1).all()
    assert np.abs(w1 - w0).max() / np.abs(w0).max() < 1e-2
    # deadband: nothing moves
    w0, w1, *_ , re, ce = _rebal(O, ri(-50, 50), ri(40, 60), ri(40, 60), 0, 0, True)
    assert np.abs(w1 - w0).max() == 0 and (re == 0).all()
    # EXP_MIN floor: -4 + -4 ticks down to -8 at most once per side
    w0, w1, *_ , re, ce = _rebal(O, ri(-5, 5), ri(-5, 5), ri(-5, 5), -8, -8, True)
    assert np.abs(w1 - w0).max() == 0 and (re == -8).all() and (ce == -8).all()


def test_rebalance_tickup_unbiased(oracle):
    O = oracle
    rng = np.random.default_rng(11)
    N, K = 4, 8
    sf = rng.integers(-3000, 3000, (N, K))
    ss = np.full((N, K), 120)
    vs = rng.integers(90, 127, (N, K))
    acc = 0.0
    T = 2000
    for s in range(T):
        w0, w1, *_ = _rebal(O, sf, ss, vs, 0, 0, False, seed=s)
        acc = acc + w1
    assert np.abs(acc / T - w0).max() / np.abs(w0).max() < 2e-3


# --------------------------------------------------------------- v-hat EMA


def test_vhat_matches_float64(oracle):
    rng = np.random.default_rng(12)
    for N, K in [(70, 130), (300, 65)]:
        g = (rng.standard_normal((N, K)) * 1e-3).astype(np.float32)
        gb = oracle.f32_to_bf16_bits_array(g)
        gd = oracle.bf16_bits_to_f32(gb).astype(np.float64)
        vr = rng.random(N).astype(np.float32) * 1e-6
        vc = rng.random(K).astype(np.float32) * 1e-6
        vr0, vc0 = vr.astype(np.float64), vc.astype(np.float64)
        svi = oracle.vhat_ema(gb, vr, vc, 0.999)
        wr = 0.999 * vr0 + 0.001 * (gd * gd).sum(1)
        wc = 0.999 * vc0 + 0.001 * (gd * gd).sum(0)
        np.testing.assert_allclose(vr, wr, rtol=2e-6)
        np.testing.assert_allclose(vc, wc, rtol=2e-6)
        assert abs(svi - 1.0 / wr.sum()) <= 2e-6 / wr.sum()


def test_vhat_exact_on_dyadic_input(oracle):
    # g = +-2^-6 everywhere: every partial sum is exact, so the result is the
    # closed form regardless of the reduction order
    N, K = 96, 200
    rng = np.random.default_rng(13)
    g = (np.where(rng.random((N, K)) < 0.5, -1.0, 1.0) * 2.0 ** -6).astype(np.float32)
    gb = oracle.f32_to_bf16_bits_array(g)
    vr = np.zeros(N, np.float32)
    vc = np.zeros(K, np.float32)
    svi = oracle.vhat_ema(gb, vr, vc, 0.5)
    np.testing.assert_array_equal(vr, np.full(N, 0.5 * K * 2.0 ** -12, np.float32))
    np.testing.assert_array_equal(vc, np.full(K, 0.5 * N * 2.0 ** -12, np.float32))
    assert svi == np.float32(1.0) / np.float32(N * 0.5 * K * 2.0 ** -12)


# ------------------------------------------------------------ load_weights


def test_load_weights_edges(oracle):
    W = np.zeros((6, 8), np.float32)
    W[0, 0] = 0.25                     # power of two: ceil(log2 + 1) = -1
    W[1, 0] = 0.25 * (1 + 2 ** -10)    # just above: 0
    W[2, 3] = 1e4                      # clamps at EXP_MAX = 7
    W[4, :] = 2.5 * 2.0 ** (-1 - 15)   # row exp -1 after max 0.25? no: max = 2.5*2^-16
    W[5, 1] = -0.75
    p, re, ce = oracle.load_weights(W)
    assert re.tolist()[:4] == [-1, 0, 7, -8]
    assert not ce.any()
    sf, ss, vs = oracle.unpack(p)
    assert not ss.any() and not vs.any()
    # row 0: 0.25 / 2^(-1-15) = 16384 exactly
    assert sf[0, 0] == 16384
    # row 2 saturates at int16
    assert sf[2, 3] == 32767
    # row 4: max 2.5*2^-16 -> exp = ceil(log2(2.5)-16+1) = -13 -> clamp -8: tiny mantissa,
    # 2.5*2^-16 / 2^-23 = 320 exactly
    assert re[4] == -8 and (sf[4] == 320).all()
    # round half to even: row 5 max 0.75 -> exp 1 -> scale 2^-14; W = 0.75 -> 12288
    assert re[5] == 1 and sf[5, 1] == -12288


# ------------------------------------------------------------ Muon NS5 drive


def _ns5_float64(G):
    """The Muon drive's orthogonalisation in float64 (no bf16 rounding):
    g / max(||g||, 1e-12) (exp9_muon.py:75, 82), then ns5 of that unit
    matrix (44-55), which divides by its norm + 1e-7 once more."""
    a, b, c = 3.4445, -4.7750, 2.0315
    G = G / max(np.linalg.norm(G), 1e-12)
    X = G / (np.linalg.norm(G) + 1e-7)
    tr = X.shape[0] > X.shape[1]
    if tr:
        X = X.T
    for _ in range(5):
        A = X @ X.T
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    return X.T if tr else X


def test_frob_sumsq(oracle):
    rng = np.random.default_rng(21)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((70, 300)) * 1e-2).astype(np.float32))
    gd = oracle.bf16_bits_to_f32(g).astype(np.float64)
    assert abs(oracle.frob_sumsq(g) - (gd * gd).sum()) <= 1e-6 * (gd * gd).sum()
    # dyadic: exact whatever the order
    d = oracle.f32_to_bf16_bits_array(np.full((33, 500), -2.0 ** -5, np.float32))
    assert oracle.frob_sumsq(d) == np.float32(33 * 500 * 2.0 ** -10)


def _ns5_bf16_numpy(oracle, G, gamma):
    """The same bf16 rounding points as the oracle, written independently in
    numpy (float64 products, float32 elementwise)."""
    def rb(x):
        return oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits_array(np.asarray(x, np.float32))).astype(np.float64)
    a, b, c = np.float32(3.4445), np.float32(-4.7750), np.float32(2.0315)
    norm = np.float32(np.sqrt(np.float32((G * G).sum())))
    n = max(norm, np.float32(1e-12))
    den = np.float32(n * np.float32(np.float32(norm / n) + np.float32(1e-7)))
    X = rb(G.astype(np.float32) / den)
    tr = X.shape[0] > X.shape[1]
    if tr:
        X = X.T.copy()
    for _ in range(5):
        A = rb(X @ X.T)
        AA = rb(A @ A)
        B = rb(b * A.astype(np.float32) + c * AA.astype(np.float32))
        X = rb(a * X.astype(np.float32) + rb(B @ X).astype(np.float32))
    out = rb(np.float32(gamma) * X.astype(np.float32))
    return out.T if tr else out


@pytest.mark.parametrize("N,K", [(96, 160), (160, 96), (128, 128), (40, 300)])
def test_ns5_matches_independent_iterations(oracle, N, K):
    """The oracle's bf16 NS5 against (1) the same rounding points restated in
    numpy, to the products' accumulation order, and (2) the reference
    iteration in float64, to the bf16 NS5's own error (~2%).  A wrong
    coefficient, sign, operand order or missing transpose fails both."""
    rng = np.random.default_rng(N * 7 + K)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 1e-3).astype(np.float32))
    gd = oracle.bf16_bits_to_f32(g).astype(np.float64)
    gamma = np.float32(np.sqrt(np.float32(max(N, K))))
    got = oracle.bf16_bits_to_f32(oracle.muon_ns5(g, gamma)).astype(np.float64)
    em = _ns5_bf16_numpy(oracle, gd, gamma)
    # two restatements of one bf16 method differ only where a product's
    # accumulation order flips a bf16 rounding; five iterations amplify
    # such flips to ~7e-3 at most here
    assert np.linalg.norm(got - em) / np.linalg.norm(em) < 1.5e-2
    ref = gamma * _ns5_float64(gd)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 4e-2


def test_ns5_small_norm_input_is_normalised(oracle):
    """A gradient of norm ~1e-7 still enters NS5 as a unit matrix: the drive
    divides by max(||g||, 1e-12) before ns5 adds its 1e-7 (exp9_muon.py:75,
    82, 47).  Dividing once by ||g|| + 1e-7 would halve the input here and
    leave the five iterations short of the quintic's band."""
    rng = np.random.default_rng(31)
    N, K = 64, 192
    g = rng.standard_normal((N, K))
    g *= 1e-7 / np.linalg.norm(g)
    gb = oracle.f32_to_bf16_bits_array(g.astype(np.float32))
    gd = oracle.bf16_bits_to_f32(gb).astype(np.float64)
    assert 0.9e-7 < np.linalg.norm(gd) < 1.1e-7
    gamma = np.float32(np.sqrt(np.float32(K)))
    got = oracle.bf16_bits_to_f32(oracle.muon_ns5(gb, gamma)).astype(np.float64)
    ref = gamma * _ns5_float64(gd)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 4e-2
    # and it is the same drive as for the same direction at unit scale
    g1 = oracle.f32_to_bf16_bits_array((gd / np.linalg.norm(gd)).astype(np.float32))
    one = oracle.bf16_bits_to_f32(oracle.muon_ns5(g1, gamma)).astype(np.float64)
    assert np.linalg.norm(got - one) / np.linalg.norm(one) < 2e-2


def test_ns5_norm_below_clamp_is_renormalised(oracle):
    """Below the drive's clamp (||g|| < 1e-12) g / 1e-12 has norm < 1, and
    ns5's own division by (that norm + 1e-7) brings it back to unit norm
    (exp9_muon.py:75, 47).  A single denominator max(||g||, 1e-12) * (1 +
    1e-7) would feed NS5 a matrix of norm ~0.01 here, whose five iterations
    stay far from the quintic's band; the float64 two-step reference and the
    unit-scale drive of the same direction both catch that."""
    rng = np.random.default_rng(37)
    N, K = 64, 192
    g = rng.standard_normal((N, K))
    g *= 1e-14 / np.linalg.norm(g)
    gb = oracle.f32_to_bf16_bits_array(g.astype(np.float32))
    gd = oracle.bf16_bits_to_f32(gb).astype(np.float64)
    assert 0.9e-14 < np.linalg.norm(gd) < 1.1e-14
    gamma = np.float32(np.sqrt(np.float32(K)))
    got = oracle.bf16_bits_to_f32(oracle.muon_ns5(gb, gamma)).astype(np.float64)
    ref = gamma * _ns5_float64(gd)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 4e-2
    em = _ns5_bf16_numpy(oracle, gd, gamma)
    assert np.linalg.norm(got - em) / np.linalg.norm(em) < 1.5e-2
    g1 = oracle.f32_to_bf16_bits_array((gd / np.linalg.norm(gd)).astype(np.float32))
    one = oracle.bf16_bits_to_f32(oracle.muon_ns5(g1, gamma)).astype(np.float64)
    assert np.linalg.norm(got - one) / np.linalg.norm(one) < 2e-2


def test_ns5_singular_values_in_quintic_band(oracle):
    """NS5 with the Muon quintic maps every singular value of a full-rank
    input into roughly [0.68, 1.14] (semi-orthogonal up to that band);
    the spectral norm of the drive is then ~gamma."""
    rng = np.random.default_rng(5)
    for N, K in [(64, 256), (256, 64)]:
        g = oracle.f32_to_bf16_bits_array(rng.standard_normal((N, K)).astype(np.float32))
        gamma = np.sqrt(max(N, K))
        X = oracle.bf16_bits_to_f32(oracle.muon_ns5(g, gamma)).astype(np.float64) / gamma
        sv = np.linalg.svd(X, compute_uv=False)
        assert sv.min() > 0.6 and sv.max() < 1.25, (sv.min(), sv.max())


def test_ns5_transpose_and_scale(oracle):
    rng = np.random.default_rng(8)
    g = rng.standard_normal((48, 200)).astype(np.float32) * 1e-3
    gb = oracle.f32_to_bf16_bits_array(g)
    gt = oracle.f32_to_bf16_bits_array(np.ascontiguousarray(g.T))
    o = oracle.bf16_bits_to_f32(oracle.muon_ns5(gb, 1.0)).astype(np.float64)
    ot = oracle.bf16_bits_to_f32(oracle.muon_ns5(gt, 1.0)).astype(np.float64)
    assert np.linalg.norm(o - ot.T) / np.linalg.norm(o) < 1e-2
    # a power-of-two scale of g changes nothing but the norm's exponent
    g4 = oracle.f32_to_bf16_bits_array(g * 4.0)
    np.testing.assert_array_equal(oracle.muon_ns5(g4, 1.0), oracle.muon_ns5(gb, 1.0))


# ---------------------------------------------------------------- coherence meter

def _coh_f32(packed, C):
    p = packed.astype(np.int64)
    sf = (packed >> 16).astype(np.float32)
    ss = ((packed << 16) >> 24).astype(np.int64)
    vs = ((packed << 24) >> 24).astype(np.int64)
    sig = np.float32(C) * ((ss - vs) * 128).astype(np.float32)
    noise = sf - sig
    sig2 = sig * sig
    return sig2 / ((sig2 + noise * noise) + np.float32(1e-30))


def test_coherence_sum_closed_forms(oracle):
    """Zero state -> 0; s_fast = 0 with s_slow != v_slow -> every word's gain
    is exactly 1/2 (noise = -sig); s_slow == v_slow -> 0 whatever s_fast."""
    C = 0.018036072144288578
    assert oracle.coherence_sum(np.zeros((7, 300), np.int32), C) == 0.0
    rng = np.random.default_rng(0)
    ss = rng.integers(-128, 128, (64, 200))
    vs = (ss + rng.integers(1, 100, (64, 200)) + 128) % 256 - 128
    assert (ss != vs).all()
    words = (((ss & 0xFF) << 8) | (vs & 0xFF)).astype(np.int32)
    assert oracle.coherence_sum(words, C) == np.float32(0.5 * words.size)
    sf = rng.integers(-32768, 32768, (64, 200))
    words = (((sf & 0xFFFF) << 16) | ((ss & 0xFF) << 8) | (ss & 0xFF)).astype(np.uint32).view(np.int32)
    assert oracle.coherence_sum(words, C) == 0.0


def test_coherence_sum_order_and_value(oracle):
    """A single block smaller than the lane count is the halving tree of the
    per-word gains; larger inputs agree with a float64 sum of the same float32
    gains (the association only moves low bits)."""
    C = 0.018036072144288578
    rng = np.random.default_rng(1)
    small = rng.integers(-2 ** 31, 2 ** 31, (3, 50), dtype=np.int64).astype(np.int32)
    g = np.zeros(256, np.float32)
    g[:small.size] = _coh_f32(small, C).ravel()
    for h in (128, 64, 32, 16, 8, 4, 2, 1):
        g[:h] = g[:h] + g[h:2 * h]
    assert oracle.coherence_sum(small, C) == g[0]
    big = rng.integers(-2 ** 31, 2 ** 31, (300, 777), dtype=np.int64).astype(np.int32)
    want = _coh_f32(big, C).astype(np.float64).sum()
    got = float(oracle.coherence_sum(big, C))
    assert abs(got - want) <= 1e-5 * want


def test_materialize_gated_closed_forms(oracle):
    """fast_gain = 1 is the live weight and 0 the consolidated one exactly
    (every partial sum is an integer below 2^24); other gains follow the
    reference's float32 expression ((128 ss + g sf) + 128 vs) * 2^e, RNE."""
    rng = np.random.default_rng(4)
    N, K = 40, 70
    packed = rng.integers(-2 ** 31, 2 ** 31, (N, K), dtype=np.int64).astype(np.int32)
    re = rng.integers(-8, 8, N).astype(np.int8)
    ce = rng.integers(-8, 8, K).astype(np.int8)
    np.testing.assert_array_equal(oracle.materialize_gated(packed, re, ce, 1.0),
                                  oracle.materialize(packed, re, ce))
    np.testing.assert_array_equal(oracle.materialize_gated(packed, re, ce, 0.0),
                                  oracle.materialize(packed, re, ce, consolidated=True))
    g = np.float32(0.37)
    sf = (packed >> 16).astype(np.float32)
    ss = ((packed << 16) >> 24).astype(np.float32)
    vs = ((packed << 24) >> 24).astype(np.float32)
    m = (ss * np.float32(128) + g * sf) + vs * np.float32(128)
    e = (re.astype(np.int32)[:, None] + ce.astype(np.int32)[None, :] - 15).astype(np.float32)
    v = (m * np.exp2(e).astype(np.float32)).astype(np.float32)
    want = oracle.f32_to_bf16_bits_array(v)
    np.testing.assert_array_equal(oracle.materialize_gated(packed, re, ce, 0.37), want)


# ---------------------------------------------------------------- gradient noise

def test_iso_draws_match_float64_box_muller(oracle):
    """The isotropic stream takes four draws from each Philox4x32-10 block
    (counter (b, 0, 0, 0), key (seed, 0x6E6F6973)): words (0, 1) and (2, 3)
    are Box-Muller pairs, each giving its cos and then its sin draw.  The
    fixed-order float32 log2 / sqrt / sincos(2 pi u) agree with float64 to
    ~1e-6 of the draw's scale, in all four quadrants of the angle."""
    seed = -12345
    z = oracle.iso_draws(seed, 4 * 1200)
    quads = set()
    for b in range(0, 1200, 7):
        c = oracle.philox4x32_10([b, 0, 0, 0], [seed & 0xFFFFFFFF, oracle.TAG_ISO])
        for p in (0, 1):
            u1 = ((int(c[2 * p]) >> 8) + 1) * 2.0 ** -24
            u2 = (int(c[2 * p + 1]) >> 8) * 2.0 ** -24
            quads.add(int(u2 * 4))
            r = np.sqrt(-2.0 * np.log(u1))
            for k, want in enumerate((r * np.cos(2.0 * np.pi * u2), r * np.sin(2.0 * np.pi * u2))):
                got = float(z[4 * b + 2 * p + k])
                assert abs(got - want) <= 4e-6 * max(1.0, abs(want)), (b, p, k, got, want)
        # the block's first draw is the one-draw form on the same block
        assert z[4 * b] == oracle.normal_draw_tag(seed, b, oracle.TAG_ISO)
    assert quads == {0, 1, 2, 3}


def test_iso_draw_statistics(oracle):
    z = oracle.iso_draws(7, 400000).astype(np.float64)
    assert abs(z.mean()) < 5e-3 and abs(z.std() - 1.0) < 5e-3
    assert abs((np.abs(z) > 2.0).mean() - 0.0455) < 2e-3
    assert abs(np.mean(z ** 4) - 3.0) < 5e-2          # Gaussian kurtosis
    q = z.reshape(-1, 4)
    for a, b in ((0, 1), (2, 3), (0, 2), (1, 3)):     # the cos/sin pairs and the two pairs
        assert abs(np.corrcoef(q[:, a], q[:, b])[0, 1]) < 1e-2
        assert abs(np.corrcoef(q[:, a] ** 2, q[:, b] ** 2)[0, 1]) < 2e-2
    z2 = oracle.iso_draws(8, 400000).astype(np.float64)
    assert abs(np.corrcoef(z, z2)[0, 1]) < 1e-2       # streams of different seeds


def test_iso_noise_closed_forms(oracle):
    rng = np.random.default_rng(2)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((37, 300)) * 1e-3).astype(np.float32))
    np.testing.assert_array_equal(oracle.iso_noise(g, 0.0, 5), g)           # sigma = 0
    zero = np.zeros((20, 50), np.uint16)
    np.testing.assert_array_equal(oracle.iso_noise(zero, 0.3, 5), zero)     # ||g|| = 0
    out = oracle.iso_noise(g, 0.1, 5)
    gf = oracle.bf16_bits_to_f32(g).astype(np.float64)
    d = oracle.bf16_bits_to_f32(out).astype(np.float64) - gf
    # the added noise has norm sigma ||g|| (up to the bf16 rounding of g + noise)
    assert abs(np.linalg.norm(d) / np.linalg.norm(gf) - 0.1) < 5e-3
    # and follows the stream: the same salt draws the same noise, another does not
    np.testing.assert_array_equal(oracle.iso_noise(g, 0.1, 5), out)
    assert (oracle.iso_noise(g, 0.1, 6) != out).any()


def test_token_draws_are_the_tagged_stream(oracle):
    """The per-token draws are Box-Muller (words 0 and 1, cos output) on
    Philox block (m, 0, 0, 0) under the second key word 0x5369676D, and the
    token sum is their fixed-order float32 total."""
    seed = 4242
    eps = oracle.token_draws(seed, 3000)
    for m in range(0, 3000, 53):
        c = oracle.philox4x32_10([m, 0, 0, 0], [seed, oracle.TAG_TOKEN])
        u1 = ((int(c[0]) >> 8) + 1) * 2.0 ** -24
        u2 = (int(c[1]) >> 8) * 2.0 ** -24
        want = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        assert abs(float(eps[m]) - want) <= 4e-6 * max(1.0, abs(want))
    assert not np.array_equal(eps[:100], oracle.iso_draws(seed, 400)[::4])
    for M in (1, 7, 8192, 8193, 20000):
        e = oracle.token_draws(seed, M).astype(np.float64)
        assert abs(float(oracle.token_sum(seed, M)) - e.sum()) < 1e-5 * max(1.0, np.abs(e).sum())
    assert float(oracle.token_sum(seed, 1)) == float(oracle.token_draws(seed, 1)[0])


def test_sigmag_combine_closed_forms(oracle):
    rng = np.random.default_rng(3)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((40, 70)) * 1e-2).astype(np.float32))
    P = oracle.f32_to_bf16_bits_array((rng.standard_normal((40, 70)) * 1e-2).astype(np.float32))
    np.testing.assert_array_equal(oracle.sigmag_combine(g, P, 1.5, 64, 0.0), g)   # sigma = 0
    # P = S g / M exactly (M a power of two, S = M): the centred draw is zero
    np.testing.assert_array_equal(oracle.sigmag_combine(g, g, 64.0, 64, 0.3), g)
    # otherwise the added part has norm sigma ||g|| along P - S g / M
    out = oracle.sigmag_combine(g, P, 3.0, 16, 0.2)
    gf = oracle.bf16_bits_to_f32(g).astype(np.float64)
    d = oracle.bf16_bits_to_f32(out).astype(np.float64) - gf
    z = oracle.bf16_bits_to_f32(P).astype(np.float64) - 3.0 * gf / 16
    assert abs(np.linalg.norm(d) / np.linalg.norm(gf) - 0.2) < 5e-3
    assert np.dot(d.ravel(), z.ravel()) / (np.linalg.norm(d) * np.linalg.norm(z)) > 0.999


def test_sigmag_draw_is_centred_per_token_gradients(oracle):
    """Brute force on a tiny layer: the draw the library forms from the
    scaled dy, the bf16 product and the token sum points along
    sum_m eps_m (g_m - mean_m g_m), g_m = dy_m^T x_m, the definition of a
    Sigma_g-shaped sample."""
    rng = np.random.default_rng(9)
    M, N, K, seed, sigma = 24, 12, 10, 77, 0.5
    dy = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32)))
    x = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32)))
    eps = oracle.token_draws(seed, M)
    gm = np.einsum("mn,mk->mnk", dy.astype(np.float64), x.astype(np.float64))
    want = np.einsum("m,mnk->nk", eps.astype(np.float64), gm - gm.mean(axis=0))
    g_bits = oracle.f32_to_bf16_bits_array(gm.sum(axis=0).astype(np.float32))
    dyt = oracle.bf16_bits_to_f32(oracle.f32_to_bf16_bits_array((eps[:, None] * dy).astype(np.float32)))
    P_bits = oracle.f32_to_bf16_bits_array((dyt.astype(np.float64).T @ x.astype(np.float64)).astype(np.float32))
    out = oracle.sigmag_combine(g_bits, P_bits, oracle.token_sum(seed, M), M, sigma)
    gf = oracle.bf16_bits_to_f32(g_bits).astype(np.float64)
    d = oracle.bf16_bits_to_f32(out).astype(np.float64) - gf
    cos = np.dot(d.ravel(), want.ravel()) / (np.linalg.norm(d) * np.linalg.norm(want))
    assert cos > 0.999, cos
    assert abs(np.linalg.norm(d) / np.linalg.norm(gf) - sigma) < 1e-2
