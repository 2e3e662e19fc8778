"""GPU parity of every kernel of the packed path, through the C ABI.

Integer / byte results (packed words, exponents, watermarks, bf16 decodes,
coh_pre, v-hat) must be bit-exact against the CPU oracle and, where the
reference's own golden vectors exist, against those.  GEMM outputs must be
within rel-L2 <= 1e-2 of an fp32 dense product on the same bf16 operands.
"""
import glob
import os
import zlib

import numpy as np
import pytest
import torch

from gpu_util import DEV, dev, host, rand_grad_bits, rand_state, rel_l2, sync

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(autouse=True)
def _reset_globals():
    from concord_amd import packed_b as pb
    yield
    pb.set_fixed_coh(True)
    pb.set_gate_gain(1.0)
    pb.set_ratio_coh(False)
    pb.set_ratio_coh_floors(0.9, 0.999)
    pb.set_prototype_semantics(False)
    for t in pb._CONSOLIDATE_FLAGS.values():
        t.fill_(1)
    for t in pb._V_BC_BUFS.values():
        t.fill_(1.0)


def _set_salt(salt_next):
    from concord_amd import packed_b as pb
    pb._get_step_counter(DEV).fill_(int(salt_next) - 1)


# ---------------------------------------------------------------- decode


@pytest.mark.parametrize("N,K", [(37, 93), (256, 2048), (5, 2049), (300, 130)])
@pytest.mark.parametrize("consolidated", [False, True])
def test_materialize(oracle, N, K, consolidated):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N * 7 + K)
    packed, re, ce = rand_state(rng, N, K, sf=(-32768, 32768), exp=(-8, 7), col=(-8, 7))
    out = torch.empty((N, K), dtype=torch.bfloat16, device=DEV)
    pb.materialize_packed_bf16(dev(packed), dev(re), dev(ce), out, consolidated=consolidated)
    np.testing.assert_array_equal(host(out), oracle.materialize(packed, re, ce, consolidated=consolidated))


def test_materialize_strided(oracle):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(1)
    N, K = 40, 100
    big, re, ce = rand_state(rng, N, K + 13, exp=(-8, 7), col=(-8, 7))
    ce = ce[:K].copy()
    pk = dev(big)[:, :K]
    out_full = torch.zeros((N, K + 5), dtype=torch.bfloat16, device=DEV)
    out = out_full[:, :K]
    from concord_amd import _lib as C
    red, ced = dev(re), dev(ce)   # keep the device copies alive across the launch
    C.check(C.lib().concord_materialize(C.ptr(pk), pk.stride(0), C.ptr(red), C.ptr(ced), N, K,
                                        15, 0, C.ptr(out), out.stride(0), C.stream_of(DEV)), "mat")
    sync()
    np.testing.assert_array_equal(host(out), oracle.materialize(np.ascontiguousarray(big[:, :K]), re, ce))


# ---------------------------------------------------------------- update


def _adamw_flags_from_fixture(pb, z):
    s = lambda k: int(z["s_" + k])  # noqa: E731
    pb.set_fixed_coh(bool(s("fixed_coh")))
    pb.set_gate_gain(float(z["s_gate_gain"]))
    pb.set_ratio_coh(bool(s("ratio_coh")))
    pb.set_ratio_coh_floors(float(z["s_chase_floor"]), float(z["s_leak_floor"]))
    pb.set_prototype_semantics(bool(s("proto")))
    pb._get_consolidate_flag(DEV).fill_(s("consolidate"))
    pb._v_bc_buf(DEV).fill_(float(z["s_v_bc"]))


ADAMW_CASES = sorted(os.path.basename(p)[6:-4] for p in glob.glob(os.path.join(GOLD, "adamw_*.npz")))


@pytest.mark.parametrize("case", ADAMW_CASES)
def test_apply_adamw_matches_reference_golden(oracle, case):
    """GPU update on the reference's own inputs == the reference's own outputs."""
    from concord_amd import packed_b as pb
    z = np.load(os.path.join(GOLD, f"adamw_{case}.npz"))
    N, K = z["packed"].shape
    _adamw_flags_from_fixture(pb, z)
    _set_salt(int(z["s_salt"]))
    pk = dev(z["packed"])
    wbuf = torch.zeros((N, K), dtype=torch.bfloat16, device=DEV)
    rm = torch.zeros(N, dtype=torch.int32, device=DEV)
    cm = torch.zeros(K, dtype=torch.int32, device=DEV)
    cp = dev(z["coh_pre"].reshape(N, K)) if z["coh_pre"].size else None
    pb.apply_packed_adamw(
        pk, dev(z["grad"]), wbuf, dev(z["row_exp"]), dev(z["col_exp"]), rm, cm,
        lr=float(z["s_lr"]), alpha=float(z["s_alpha"]), beta1=float(z["s_beta1"]),
        weight_decay=float(z["s_weight_decay"]), eps=float(z["s_eps"]), step_cap=float(z["s_step_cap"]),
        v_scale=float(z["s_v_scale"]), gf_consol=float(z["s_gf_consol"]),
        drift_cancel_C=float(z["s_drift_cancel_C"]), alpha_v_fast=float(z["s_alpha_v_fast"]),
        wd_sv=float(z["s_wd_sv"]), wd_sf=float(z["s_wd_sf"]),
        mass_preserve=bool(int(z["s_mass_preserve"])), apply_chase=bool(int(z["s_apply_chase"])),
        track_rebalance=bool(int(z["s_track"])), v_row=dev(z["v_row"]), v_col=dev(z["v_col"]),
        sum_v_inv=dev(z["sum_v_inv"]), gf_trust_delta_sq=float(z["s_gf_trust_delta_sq"]), coh_pre=cp)
    sync()
    np.testing.assert_array_equal(host(pk), z["packed_out"])
    np.testing.assert_array_equal(host(rm), z["row_max"])
    np.testing.assert_array_equal(host(cm), z["col_max"])
    if cp is not None:
        np.testing.assert_array_equal(host(cp), z["coh_pre_out"].reshape(N, K))
    if int(z["s_consolidate"]) == 1 or not int(z["s_proto"]):
        want = oracle.materialize(z["packed_out"], z["row_exp"], z["col_exp"])
        np.testing.assert_array_equal(host(wbuf), want)
    else:
        assert not host(wbuf).any()


FLAG_SETS = {
    "bare": dict(cohpre=True),
    "winner": dict(ratio=True, gf_consol=50.0),
    "proto_accum": dict(ratio=True, gf_consol=50.0, proto=True, consolidate=0, beta1=0.1),
    "proto_cons": dict(ratio=True, gf_consol=30.0, proto=True, consolidate=1, beta1=0.1, v_bc=1.5),
    "wd_all": dict(cohpre=True, fixed=False, weight_decay=0.02, wd_sv=0.3, wd_sf=0.2, beta1=0.05,
                   v_scale=1.0, gate_gain=0.7, eps=1.0),
    "muon": dict(ratio=True, gf_consol=10.0, muon=True),
    "pow": dict(cohpre=True, precond_p=0.3),
    "sgdlike": dict(precond_p=0.0, trust=0.0, chase=False, track=False, mp=False),
    # v-hat spread over 60 decades (and exact zeros) with eps = 1e-30: the
    # square root's argument falls on both sides of 2^-96 within one wave
    "winner_tiny_v": dict(ratio=True, gf_consol=50.0, eps=1e-30, vspread=True),
    "bare_tiny_v": dict(cohpre=True, eps=1e-30, vspread=True),
    "wd_tiny_v": dict(cohpre=True, fixed=False, weight_decay=0.02, wd_sv=0.3, eps=1e-30, vspread=True),
}


@pytest.mark.parametrize("name", sorted(FLAG_SETS))
@pytest.mark.parametrize("N,K", [(130, 300), (512, 1280), (33, 1030)])
def test_apply_adamw_matches_oracle(oracle, name, N, K):
    from concord_amd import packed_b as pb
    O = oracle
    f = FLAG_SETS[name]
    rng = np.random.default_rng(zlib.crc32(f"{name}-{N}-{K}".encode()))
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-3, 3))
    g = rand_grad_bits(rng, N, K)
    vr = (rng.random(N) * 1e-3 + 1e-7).astype(np.float32)
    vc = (rng.random(K) * 1e-3 + 1e-7).astype(np.float32)
    if f.get("vspread"):
        vr = (10.0 ** -rng.uniform(0, 30, N)).astype(np.float32)
        vc = (10.0 ** -rng.uniform(0, 30, K)).astype(np.float32)
        vc[::7] = 0.0
    svi = np.array([1.0 / vr.sum()], np.float32)
    cp = rng.random((N, K)).astype(np.float32) if f.get("cohpre") else None
    salt = int(rng.integers(-2 ** 31 + 1, 2 ** 31))
    lr = 7e-4
    pb.set_fixed_coh(f.get("fixed", True))
    pb.set_gate_gain(f.get("gate_gain", 1.0))
    pb.set_ratio_coh(f.get("ratio", False))
    pb.set_ratio_coh_floors(0.6, 0.8)
    pb.set_prototype_semantics(f.get("proto", False))
    pb._get_consolidate_flag(DEV).fill_(f.get("consolidate", 1))
    pb._v_bc_buf(DEV).fill_(f.get("v_bc", 1.0))
    _set_salt(salt)
    kw = dict(alpha=0.1, beta1=f.get("beta1", 0.0), weight_decay=f.get("weight_decay", 0.0),
              eps=f.get("eps", 1e-10), step_cap=10.0, v_scale=f.get("v_scale", 0.0),
              precond_p=f.get("precond_p", 0.5), gf_consol=f.get("gf_consol", 0.0),
              drift_cancel_C=0.018036072144288578, alpha_v_fast=0.001, wd_sv=f.get("wd_sv", 0.0),
              wd_sf=f.get("wd_sf", 0.0), mass_preserve=f.get("mp", True),
              apply_chase=f.get("chase", True), track_rebalance=f.get("track", True),
              gf_trust_delta_sq=f.get("trust", 1.0))
    pk, wb = dev(packed), torch.zeros((N, K), dtype=torch.bfloat16, device=DEV)
    rm = torch.zeros(N, dtype=torch.int32, device=DEV)
    cm = torch.zeros(K, dtype=torch.int32, device=DEV)
    cpd = dev(cp) if cp is not None else None
    pb.apply_packed_adamw(pk, dev(g), wb, dev(re), dev(ce), rm, cm, lr=lr, v_row=dev(vr),
                          v_col=dev(vc), sum_v_inv=dev(svi), coh_pre=cpd,
                          drive_muon=f.get("muon", False), **kw)
    sync()
    # oracle
    flags = O.EMIT_WEIGHT
    for key, bit in [("mp", O.MASS_PRESERVE), ("chase", O.APPLY_CHASE), ("track", O.TRACK_REBALANCE)]:
        if f.get(key, True):
            flags |= bit
    if kw["gf_trust_delta_sq"] > 0:
        flags |= O.GF_TRUST_REGION
    if kw["gf_consol"] > 0:
        flags |= O.GF_CONSOLIDATION
    if cp is not None:
        flags |= O.COHPRE
    if f.get("fixed", True):
        flags |= O.FIXED_COH
    if f.get("ratio", False):
        flags |= O.RATIO_COH
    if f.get("proto", False):
        flags |= O.PROTO_CONSF
    if f.get("muon", False):
        flags |= O.MUON
    P = O.UpdateParams(alpha=kw["alpha"], beta1=kw["beta1"], weight_decay=kw["weight_decay"],
                       step_cap=10.0, v_scale=kw["v_scale"], precond_p=kw["precond_p"],
                       gf_consol=kw["gf_consol"], drift_cancel_C=kw["drift_cancel_C"],
                       alpha_v_fast=0.001, wd_sv=kw["wd_sv"], wd_sf=kw["wd_sf"],
                       gf_trust_delta_sq=kw["gf_trust_delta_sq"], gate_gain=f.get("gate_gain", 1.0),
                       mantissa_bias=15)
    S = O.UpdateScalars(lr=lr, eps=kw["eps"], chase_floor=0.6, leak_floor=0.8, v_bc=f.get("v_bc", 1.0),
                        salt=salt, consolidate=f.get("consolidate", 1))
    opk = packed.copy()
    ow = np.zeros((N, K), np.uint16)
    orm = np.zeros(N, np.int32)
    ocm = np.zeros(K, np.int32)
    ocp = cp.copy() if cp is not None else None
    O.apply_adamw(opk, g, ow, re, ce, orm, ocm, vr, vc, float(svi[0]), ocp, P, S, flags)
    np.testing.assert_array_equal(host(pk), opk)
    np.testing.assert_array_equal(host(wb), ow)
    np.testing.assert_array_equal(host(rm), orm)
    np.testing.assert_array_equal(host(cm), ocm)
    if cp is not None:
        np.testing.assert_array_equal(host(cpd), ocp)
    assert (opk != packed).any()


def test_tall_layer_beyond_grid_y(oracle):
    """A layer of 65537 x 64 words: launches keep grid.y at most 65535 (the
    materialize kernels stride their rows over it), and materialize and the
    packed update stay bit-exact against the oracle on every row."""
    from concord_amd import packed_b as pb
    O = oracle
    N, K = 65537, 64
    rng = np.random.default_rng(65537)
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-2, 2))
    pk, red, ced = dev(packed), dev(re), dev(ce)
    for cons in (False, True):
        w = torch.empty((N, K), dtype=torch.bfloat16, device=DEV)
        pb.materialize_packed_bf16(pk, red, ced, w, consolidated=cons)
        sync()
        np.testing.assert_array_equal(host(w), O.materialize(packed, re, ce, consolidated=cons))
    g = rand_grad_bits(rng, N, K)
    vr = (rng.random(N) * 1e-3 + 1e-7).astype(np.float32)
    vc = (rng.random(K) * 1e-3 + 1e-7).astype(np.float32)
    svi = np.array([1.0 / vr.sum()], np.float32)
    _set_salt(77)
    pb.set_ratio_coh(True)
    pb.set_ratio_coh_floors(0.9, 0.999)
    rm = torch.zeros(N, dtype=torch.int32, device=DEV)
    cm = torch.zeros(K, dtype=torch.int32, device=DEV)
    pb.apply_packed_adamw(pk, dev(g), None, red, ced, rm, cm, lr=5e-4, eps=1e-10, gf_consol=50.0,
                          v_scale=0.0, mass_preserve=True, v_row=dev(vr), v_col=dev(vc), sum_v_inv=dev(svi),
                          gf_trust_delta_sq=1.0, coh_pre=None)
    sync()
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0, precond_p=0.5,
                       gf_consol=50.0, drift_cancel_C=0.018036072144288578, alpha_v_fast=0.001, wd_sv=0.0,
                       wd_sf=0.0, gf_trust_delta_sq=1.0, gate_gain=1.0, mantissa_bias=15)
    S = O.UpdateScalars(lr=5e-4, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0, salt=77,
                        consolidate=1)
    flags = (O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH
             | O.RATIO_COH | O.GF_CONSOLIDATION)
    opk = packed.copy()
    orm = np.zeros(N, np.int32)
    ocm = np.zeros(K, np.int32)
    O.apply_adamw(opk, g, None, re, ce, orm, ocm, vr, vc, float(svi[0]), None, P, S, flags)
    np.testing.assert_array_equal(host(pk), opk)
    np.testing.assert_array_equal(host(rm), orm)
    np.testing.assert_array_equal(host(cm), ocm)


def test_apply_adamw_extreme_values(oracle):
    """Overflowing ticks: saturating float->int, int32 wrap, int16/int8 clamps."""
    from concord_amd import packed_b as pb
    O = oracle
    N, K = 64, 256
    rng = np.random.default_rng(5)
    packed, re, ce = rand_state(rng, N, K, sf=(-32768, 32768), exp=(-8, -8), col=(-8, -8), big_frac=0.5)
    g = O.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 1e3).astype(np.float32))
    vr = np.full(N, 1e-30, np.float32)
    vc = np.full(K, 1e-30, np.float32)
    svi = np.array([1e-10], np.float32)
    _set_salt(99)
    pk = dev(packed)
    rm = torch.zeros(N, dtype=torch.int32, device=DEV)
    cm = torch.zeros(K, dtype=torch.int32, device=DEV)
    pb.apply_packed_adamw(pk, dev(g), None, dev(re), dev(ce), rm, cm, lr=50.0, eps=1e-30,
                          step_cap=1e30, v_scale=0.0, gf_consol=0.0, mass_preserve=True,
                          v_row=dev(vr), v_col=dev(vc), sum_v_inv=dev(svi), gf_trust_delta_sq=1.0,
                          wd_sv=3.0, wd_sf=5.0)
    sync()
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=1e30, v_scale=0.0,
                       precond_p=0.5, gf_consol=0.0, drift_cancel_C=0.018036072144288578,
                       alpha_v_fast=0.001, wd_sv=3.0, wd_sf=5.0, gf_trust_delta_sq=1.0,
                       gate_gain=1.0, mantissa_bias=15)
    S = O.UpdateScalars(lr=50.0, eps=1e-30, chase_floor=0.9, leak_floor=0.999, v_bc=1.0, salt=99,
                        consolidate=1)
    opk = packed.copy()
    orm = np.zeros(N, np.int32)
    ocm = np.zeros(K, np.int32)
    O.apply_adamw(opk, g, None, re, ce, orm, ocm, vr, vc, float(svi[0]), None, P, S,
                  O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH)
    np.testing.assert_array_equal(host(pk), opk)
    np.testing.assert_array_equal(host(rm), orm)
    np.testing.assert_array_equal(host(cm), ocm)


@pytest.mark.parametrize("case", ["mp", "nomp"])
def test_apply_sgd_matches_reference_golden(oracle, case):
    from concord_amd import packed_b as pb
    z = np.load(os.path.join(GOLD, f"sgd_{case}.npz"))
    N, K = z["packed"].shape
    _set_salt(int(z["s_salt"]))
    pk = dev(z["packed"])
    wb = torch.zeros((N, K), dtype=torch.bfloat16, device=DEV)
    rm = torch.zeros(N, dtype=torch.int32, device=DEV)
    cm = torch.zeros(K, dtype=torch.int32, device=DEV)
    pb.apply_packed_sgd(pk, dev(z["grad"]), wb, dev(z["row_exp"]), dev(z["col_exp"]), rm, cm,
                        lr=float(z["s_lr"]), alpha=float(z["s_alpha"]), beta1=float(z["s_beta1"]),
                        alpha_v_fast=float(z["s_alpha_v_fast"]),
                        mass_preserve=bool(int(z["s_mass_preserve"])), track_rebalance=True)
    sync()
    np.testing.assert_array_equal(host(pk), z["packed_out"])
    np.testing.assert_array_equal(host(rm), z["row_max"])
    np.testing.assert_array_equal(host(cm), z["col_max"])
    np.testing.assert_array_equal(host(wb), oracle.materialize(z["packed_out"], z["row_exp"], z["col_exp"]))


# ---------------------------------------------------------------- rebalance


@pytest.mark.parametrize("case", ["up", "up_td", "tickdown"])
def test_rebalance_matches_reference_golden(case):
    from concord_amd import packed_b as pb
    z = np.load(os.path.join(GOLD, f"rebalance_{case}.npz"))
    pk, re, ce = dev(z["packed"]), dev(z["row_exp"]), dev(z["col_exp"])
    seed = torch.tensor([int(z["s_seed"])], dtype=torch.int32, device=DEV)
    pb.rebalance_packed(pk, re, ce, dev(z["row_max"]), dev(z["col_max"]), seed_buf=seed,
                        allow_tickdown=bool(int(z["s_allow_tickdown"])))
    sync()
    np.testing.assert_array_equal(host(pk), z["packed_out"])
    np.testing.assert_array_equal(host(re), z["row_exp_out"])
    np.testing.assert_array_equal(host(ce), z["col_exp_out"])
    assert int(host(seed)[0]) == int(z["s_seed"])


@pytest.mark.parametrize("N,K,tickdown", [(200, 700, False), (200, 700, True), (1024, 256, True),
                                          (70, 70, False)])
def test_rebalance_matches_oracle(oracle, N, K, tickdown):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + K + tickdown)
    sf = rng.integers(-3000, 3000, (N, K))
    small = rng.random(N) < 0.5
    ss = np.where(small[:, None], rng.integers(-20, 20, (N, K)), rng.integers(-100, 100, (N, K)))
    vs = np.where(small[:, None], rng.integers(-20, 20, (N, K)), rng.integers(-100, 100, (N, K)))
    for r in rng.choice(N, 5, replace=False):
        c = rng.integers(0, K)
        ss[r, c], vs[r, c] = 120, 125
    packed = oracle.pack(sf, ss, vs)
    re = rng.integers(-6, 8, N).astype(np.int8)
    ce = rng.integers(-6, 8, K).astype(np.int8)
    m = ss * 128 + sf + vs * 128
    rmax = np.abs(m).max(1).astype(np.int32)
    cmax = np.abs(m).max(0).astype(np.int32)
    hw_r = rng.integers(0, 30000, N).astype(np.int32)
    hw_c = rng.integers(0, 30000, K).astype(np.int32)
    pk, red, ced = dev(packed), dev(re), dev(ce)
    seed = torch.tensor([41], dtype=torch.int32, device=DEV)
    hr, hc = dev(hw_r), dev(hw_c)
    pb.rebalance_packed(pk, red, ced, dev(rmax), dev(cmax), seed_buf=seed, allow_tickdown=tickdown,
                        row_hwm=hr, col_hwm=hc, advance_seed=True)
    sync()
    opk, ore, oce = packed.copy(), re.copy(), ce.copy()
    oracle.rebalance(opk, ore, oce, rmax, cmax, seed=42, allow_tickdown=tickdown)
    np.testing.assert_array_equal(host(pk), opk)
    np.testing.assert_array_equal(host(red), ore)
    np.testing.assert_array_equal(host(ced), oce)
    np.testing.assert_array_equal(host(hr), np.maximum(hw_r, rmax))
    np.testing.assert_array_equal(host(hc), np.maximum(hw_c, cmax))
    assert int(host(seed)[0]) == 42
    assert (opk != packed).any()


@pytest.mark.parametrize("tickdown", [False, True])
def test_rebalance_stats_count_the_calls_ticks(oracle, tickdown):
    """The rebalance diagnostics (get_reb_stats; the counters of
    concord/packed_b.py:1161-1179) count the call's decisions: tick-ups and
    tick-downs are the rows and columns whose exponent the oracle's rebalance
    moved up or down, and a word clips when its larger int8 magnitude,
    shifted left by its row's and column's tick-down count, exceeds 127."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(77 + tickdown)
    N, K = 300, 500
    sf = rng.integers(-3000, 3000, (N, K))
    small = rng.random(N) < 0.5
    ss = np.where(small[:, None], rng.integers(-40, 40, (N, K)), rng.integers(-100, 100, (N, K)))
    vs = np.where(small[:, None], rng.integers(-40, 40, (N, K)), rng.integers(-100, 100, (N, K)))
    for r in rng.choice(N, 7, replace=False):
        c = rng.integers(0, K)
        ss[r, c], vs[r, c] = 120, 125
    packed = oracle.pack(sf, ss, vs)
    re = rng.integers(-6, 8, N).astype(np.int8)
    ce = rng.integers(-6, 8, K).astype(np.int8)
    m = ss * 128 + sf + vs * 128
    rmax = np.abs(m).max(1).astype(np.int32)
    cmax = np.abs(m).max(0).astype(np.int32)
    ca.reset_reb_stats()
    try:
        pb.rebalance_packed(dev(packed), dev(re), dev(ce), dev(rmax), dev(cmax),
                            seed_buf=torch.tensor([5], dtype=torch.int32, device=DEV), allow_tickdown=tickdown)
        sync()
        st = dict(ca.get_reb_stats())
    finally:
        pb._REB_STATS = None
    ore, oce = re.copy(), ce.copy()
    oracle.rebalance(packed.copy(), ore, oce, rmax, cmax, seed=5, allow_tickdown=tickdown)
    dr = ore.astype(int) - re.astype(int)
    dc = oce.astype(int) - ce.astype(int)
    assert st["tickup_dim"] == (dr > 0).sum() + (dc > 0).sum() > 0
    assert st["tickdown_dim"] == (dr < 0).sum() + (dc < 0).sum()
    assert (st["tickdown_dim"] > 0) == tickdown
    mag = np.maximum(np.abs(ss), np.abs(vs))
    lsh = np.maximum(0, -(dr[:, None] + dc[None, :]))
    assert st["clip_elems"] == ((mag << lsh) > 127).sum()
    assert (st["calls"], st["dim_total"], st["elem_total"]) == (1, N + K, N * K)


def test_rebalance_no_fire_leaves_words(oracle):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(3)
    packed, re, ce = rand_state(rng, 300, 500, sf=(-1000, 1000))
    pk = dev(packed)
    z = torch.zeros(300, dtype=torch.int32, device=DEV)
    zc = torch.zeros(500, dtype=torch.int32, device=DEV)
    pb.rebalance_packed(pk, dev(re), dev(ce), z, zc, allow_tickdown=False)
    sync()
    np.testing.assert_array_equal(host(pk), packed)


# ---------------------------------------------------------------- v-hat, load


@pytest.mark.parametrize("N,K", [(70, 130), (5120, 1280), (33, 1000), (1, 1)])
def test_vhat_matches_oracle(oracle, N, K):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N * K)
    g = rand_grad_bits(rng, N, K)
    vr = (rng.random(N) * 1e-4).astype(np.float32)
    vc = (rng.random(K) * 1e-4).astype(np.float32)
    vrd, vcd = dev(vr), dev(vc)
    svi = torch.zeros(1, dtype=torch.float32, device=DEV)
    rm = torch.full((N,), 7, dtype=torch.int32, device=DEV)
    cm = torch.full((K,), 7, dtype=torch.int32, device=DEV)
    salt = torch.tensor([5], dtype=torch.int32, device=DEV)
    for _ in range(2):   # twice: workspace reuse
        pb.vhat_ema(dev(g), vrd, vcd, svi, 0.999, rm, cm, salt)
        s = oracle.vhat_ema(g, vr, vc, 0.999)
    sync()
    np.testing.assert_array_equal(host(vrd), vr)
    np.testing.assert_array_equal(host(vcd), vc)
    assert host(svi)[0] == s
    assert not host(rm).any() and not host(cm).any()
    assert int(host(salt)[0]) == 7


@pytest.mark.parametrize("M,N,K", [(300, 2056, 648), (2048, 5120, 1280), (2048, 1280, 1280), (77, 130, 200),
                                   (64, 136, 4096), (8192, 640, 640)])
def test_wgrad_vhat_matches_separate_calls(oracle, M, N, K):
    """wgrad with the v-hat partials formed in its epilogue (fused path when
    the product runs unsplit on the transpose-read kernel, else the separate
    partials kernel) equals wgrad followed by vhat_ema bit for bit, and the
    v-hat equals the oracle's on the same bf16 gradient."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N + K + 11)
    dy = dev(oracle.f32_to_bf16_bits_array((rng.standard_normal((M, N)) * 1e-2).astype(np.float32)))
    x = dev(oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32)))
    vr = (rng.random(N) * 1e-6).astype(np.float32)
    vc = (rng.random(K) * 1e-6).astype(np.float32)
    outs = []
    for fused in (True, False):
        vrd, vcd = dev(vr), dev(vc)
        svi = torch.zeros(1, dtype=torch.float32, device=DEV)
        rm = torch.full((N,), 7, dtype=torch.int32, device=DEV)
        cm = torch.full((K,), 7, dtype=torch.int32, device=DEV)
        salt = torch.tensor([5], dtype=torch.int32, device=DEV)
        if fused:
            gw, gb = pb._wgrad_vhat(dy, x, vrd, vcd, svi, 0.999, rm, cm, salt, with_bias=True)
            # bias gradient formed from the same dy fragments (fp32 sums, bf16 out)
            ref_b = oracle.bf16_bits_to_f32(host(dy)).astype(np.float64).sum(0)
            assert rel_l2(oracle.bf16_bits_to_f32(host(gb)), ref_b) < 5e-3
        else:
            gw = pb._wgrad(dy, x)
            pb.vhat_ema(gw, vrd, vcd, svi, 0.999, rm, cm, salt)
        sync()
        assert not host(rm).any() and not host(cm).any() and int(host(salt)[0]) == 6
        outs.append((host(gw), host(vrd), host(vcd), host(svi)))
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(a, b)
    g = outs[0][0]
    s = oracle.vhat_ema(g, vr, vc, 0.999)
    np.testing.assert_array_equal(outs[0][1], vr)
    np.testing.assert_array_equal(outs[0][2], vc)
    assert outs[0][3][0] == s


def test_wgrad_vhat_repeated_calls(oracle):
    """Calls in a row over alternating shapes that share one workspace: the
    launch's block and ticket counters are re-armed by every call and sit at
    the same offsets for every shape, so each call's v-hat state, 1 / sum v_row
    and salt equal the oracle's on its own gradient."""
    from concord_amd import packed_b as pb
    shapes = [(2048, 5120, 1280), (300, 2056, 648), (2048, 5120, 1280), (512, 10240, 1280), (300, 2056, 648)]
    for it, (M, N, K) in enumerate(shapes):
        rng = np.random.default_rng(100 + it)
        dy = dev(oracle.f32_to_bf16_bits_array((rng.standard_normal((M, N)) * 1e-2).astype(np.float32)))
        x = dev(oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32)))
        vr = (rng.random(N) * 1e-6).astype(np.float32)
        vc = (rng.random(K) * 1e-6).astype(np.float32)
        vrd, vcd = dev(vr), dev(vc)
        svi = torch.zeros(1, dtype=torch.float32, device=DEV)
        rm = torch.full((N,), 7, dtype=torch.int32, device=DEV)
        cm = torch.full((K,), 7, dtype=torch.int32, device=DEV)
        salt = torch.tensor([it], dtype=torch.int32, device=DEV)
        gw, gb = pb._wgrad_vhat(dy, x, vrd, vcd, svi, 0.999, rm, cm, salt, with_bias=it % 2 == 0)
        sync()
        s = oracle.vhat_ema(host(gw), vr, vc, 0.999)
        np.testing.assert_array_equal(host(vrd), vr, err_msg=f"call {it}")
        np.testing.assert_array_equal(host(vcd), vc, err_msg=f"call {it}")
        assert host(svi)[0] == s, it
        assert int(host(salt)[0]) == it + 1 and not host(rm).any() and not host(cm).any()
        if gb is not None:
            ref_b = oracle.bf16_bits_to_f32(host(dy)).astype(np.float64).sum(0)
            assert rel_l2(oracle.bf16_bits_to_f32(host(gb)), ref_b) < 5e-3


def test_load_weights_matches_reference_golden():
    from concord_amd import packed_b as pb
    z = np.load(os.path.join(GOLD, "load_weights.npz"))
    N, K = z["W"].shape
    for ft, sfx in [(False, ""), (True, "_ft")]:
        pk = torch.zeros((N, K), dtype=torch.int32, device=DEV)
        re = torch.zeros(N, dtype=torch.int8, device=DEV)
        ce = torch.ones(K, dtype=torch.int8, device=DEV)
        pb.load_packed(torch.from_numpy(z["W"]), pk, re, ce, finetune=ft)
        sync()
        np.testing.assert_array_equal(host(pk), z["packed" + sfx])
        np.testing.assert_array_equal(host(re), z["row_exp" + sfx])
        np.testing.assert_array_equal(host(ce), z["col_exp" + sfx])


def test_load_weights_matches_oracle(oracle):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(11)
    N, K = 1000, 777
    W = (rng.standard_normal((N, K)) * 10.0 ** rng.uniform(-5, 2, (N, 1))).astype(np.float32)
    W[0] = 0
    W[1, 5] = 0.5
    for ft in (False, True):
        pk = torch.zeros((N, K), dtype=torch.int32, device=DEV)
        re = torch.zeros(N, dtype=torch.int8, device=DEV)
        ce = torch.zeros(K, dtype=torch.int8, device=DEV)
        pb.load_packed(torch.from_numpy(W), pk, re, ce, finetune=ft)
        sync()
        p, r, c = oracle.load_weights(W, finetune=ft)
        np.testing.assert_array_equal(host(pk), p)
        np.testing.assert_array_equal(host(re), r)


# ---------------------------------------------------------------- GEMMs

# (M, N, K).  Misaligned shapes run the generic kernel; shapes whose
# contiguous dimensions are multiples of 8 run the branch-free kernels, with
# ragged tile edges, a reduction tail, and (64, 136, 4096) a 4-way split-K.
# (M, N, K); the planner takes 192-row tiles for (2048, 1280, 1280) (forward and
# dgrad, 192 x 128 split two ways), (8192, 640, 640) (unsplit) and (1024, 2816,
# 2048) (forward 192 x 160), and splits the 640 x 640 WGRAD over 8192 tokens 8 ways
GEMM_SHAPES = [(64, 128, 64), (77, 130, 200), (256, 384, 1280), (1, 5, 3), (130, 1000, 70),
               (2048, 1280, 1280), (2048, 5120, 1280), (300, 2050, 645),
               (77, 136, 200), (300, 2056, 648), (1, 8, 8), (129, 1000, 72), (64, 136, 4096),
               (8192, 640, 640), (1024, 2816, 2048),
               # cross-attention k/v at batch 2 and 4 of 77 text tokens (M 154, 308)
               (154, 1280, 2048), (308, 1280, 2048), (308, 640, 2048)]


def _decoded(oracle, packed, re, ce):
    return oracle.bf16_bits_to_f32(oracle.materialize(packed, re, ce)).astype(np.float64)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_dqgemm_fwd(oracle, M, N, K):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N + K)
    packed, re, ce = rand_state(rng, N, K, exp=(-2, 2), col=(-2, 2))
    x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
    b = oracle.f32_to_bf16_bits_array(rng.standard_normal(N).astype(np.float32))
    y = pb._gemm_fwd(dev(x), dev(packed), dev(re), dev(ce), 15, dev(b), None)
    sync()
    W = _decoded(oracle, packed, re, ce)
    ref = oracle.bf16_bits_to_f32(x).astype(np.float64) @ W.T + oracle.bf16_bits_to_f32(b)
    got = oracle.bf16_bits_to_f32(host(y))
    assert rel_l2(got, ref) < 5e-3


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_dqgemm_dgrad(oracle, M, N, K):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M * 3 + N + K)
    packed, re, ce = rand_state(rng, N, K, exp=(-2, 2), col=(-2, 2))
    dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
    dx = pb._gemm_dgrad(dev(dy), dev(packed), dev(re), dev(ce), 15, None)
    sync()
    W = _decoded(oracle, packed, re, ce)
    ref = oracle.bf16_bits_to_f32(dy).astype(np.float64) @ W
    assert rel_l2(oracle.bf16_bits_to_f32(host(dx)), ref) < 5e-3


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES)
def test_wgrad(oracle, M, N, K):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M * 5 + N + K)
    dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
    x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
    gw = pb._wgrad(dev(dy), dev(x))
    sync()
    ref = oracle.bf16_bits_to_f32(dy).astype(np.float64).T @ oracle.bf16_bits_to_f32(x)
    assert rel_l2(oracle.bf16_bits_to_f32(host(gw)), ref) < 5e-3


@pytest.mark.parametrize("M,N,K", [(4096, 136, 200), (2048, 264, 256), (1000, 512, 128), (130, 8, 8)])
def test_wgrad_split_reduction(oracle, M, N, K):
    """Few output tiles and a long reduction: the planner splits the
    reduction and a second kernel adds the partial tiles."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + 3 * N + K)
    dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
    x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
    gw = pb._wgrad(dev(dy), dev(x))
    sync()
    ref = oracle.bf16_bits_to_f32(dy).astype(np.float64).T @ oracle.bf16_bits_to_f32(x)
    assert rel_l2(oracle.bf16_bits_to_f32(host(gw)), ref) < 5e-3


@pytest.mark.parametrize("M,N,K", [(96, 264, 320), (96, 130, 320)])
def test_dqgemm_extreme_exponents(oracle, M, N, K):
    """Row/column exponents at both ends of [EXP_MIN, EXP_MAX] (the fast
    kernels apply one side in the epilogue, the other while decoding)."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N + 7 * K)
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-8, 7))
    x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
    dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
    y = pb._gemm_fwd(dev(x), dev(packed), dev(re), dev(ce), 15, None, None)
    dx = pb._gemm_dgrad(dev(dy), dev(packed), dev(re), dev(ce), 15, None)
    sync()
    W = _decoded(oracle, packed, re, ce)
    assert rel_l2(oracle.bf16_bits_to_f32(host(y)), oracle.bf16_bits_to_f32(x).astype(np.float64) @ W.T) < 5e-3
    assert rel_l2(oracle.bf16_bits_to_f32(host(dx)), oracle.bf16_bits_to_f32(dy).astype(np.float64) @ W) < 5e-3


def test_gemm_splitk_workspace_reuse(oracle):
    """Back-to-back split-K GEMMs of different tile grids share one workspace:
    each call must find its counters zeroed whatever the previous call's
    partials overwrote (small grid first, then larger ones, then small again)."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(99)
    for (M, N, K) in [(300, 200, 130), (300, 2050, 645), (77, 130, 200), (300, 2050, 645),
                      (3000, 136, 200), (300, 2056, 648), (4096, 264, 256), (3000, 136, 200)]:
        dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
        x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
        gw = pb._wgrad(dev(dy), dev(x))
        sync()
        ref = oracle.bf16_bits_to_f32(dy).astype(np.float64).T @ oracle.bf16_bits_to_f32(x)
        assert rel_l2(oracle.bf16_bits_to_f32(host(gw)), ref) < 5e-3, (M, N, K)


@pytest.mark.parametrize("M,N,K", GEMM_SHAPES[:4] + GEMM_SHAPES[8:])
def test_bf16_weight_gemms(oracle, M, N, K):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M * 7 + N + K)
    w = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 0.05).astype(np.float32))
    x = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, K)).astype(np.float32))
    dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
    wd = dev(w)
    y = pb._gemm_fwd(dev(x), None, None, None, 15, None, wd)
    dx = pb._gemm_dgrad(dev(dy), torch.empty((N, K), dtype=torch.int32, device=DEV), None, None, 15, wd)
    sync()
    Wf = oracle.bf16_bits_to_f32(w).astype(np.float64)
    assert rel_l2(oracle.bf16_bits_to_f32(host(y)), oracle.bf16_bits_to_f32(x) @ Wf.T) < 5e-3
    assert rel_l2(oracle.bf16_bits_to_f32(host(dx)), oracle.bf16_bits_to_f32(dy) @ Wf) < 5e-3


def test_bias_grad(oracle):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(17)
    for M, N in [(300, 70), (4096, 1280), (1, 3)]:
        dy = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, N)).astype(np.float32))
        db = pb._bias_grad(dev(dy))
        sync()
        ref = oracle.bf16_bits_to_f32(dy).astype(np.float64).sum(0)
        assert rel_l2(oracle.bf16_bits_to_f32(host(db)), ref) < 5e-3


# ---------------------------------------------------------------- layer


def _oracle_step(oracle, layer_state, grad_bits, lr, salt, flags, coh_pre=None, chase=0.9, leak=0.999,
                 gf_consol=0.0):
    O = oracle
    pk, re, ce, vr, vc = layer_state
    N, K = pk.shape
    svi = O.vhat_ema(grad_bits, vr, vc, 0.999)
    rm = np.zeros(N, np.int32)
    cm = np.zeros(K, np.int32)
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0,
                       precond_p=0.5, gf_consol=gf_consol, drift_cancel_C=0.018036072144288578,
                       alpha_v_fast=0.001, wd_sv=0.0, wd_sf=0.0, gf_trust_delta_sq=1.0,
                       gate_gain=1.0, mantissa_bias=15)
    S = O.UpdateScalars(lr=lr, eps=1e-10, chase_floor=chase, leak_floor=leak, v_bc=1.0, salt=salt,
                        consolidate=1)
    O.apply_adamw(pk, grad_bits, None, re, ce, rm, cm, vr, vc, svi, coh_pre, P, S, flags)
    return rm, cm


@pytest.mark.parametrize("winner", [False, True])
def test_layer_config1_bit_exact(oracle, winner):
    """Config 1: 768->768 layer, Kaiming-uniform init (seed 0), x ~ N(0,1) [4096, 768],
    grad_y ~ N(0, 1e-2) (std), lr 5e-4: forward, backward (fused update), rebalance;
    packed words and consolidated_weight() bit-exact vs the oracle fed the same
    bf16 gradient."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    O = oracle
    torch.manual_seed(0)
    W0 = torch.nn.init.kaiming_uniform_(torch.empty(768, 768), a=5 ** 0.5)
    x = torch.randn(4096, 768)
    gy = torch.randn(4096, 768) * 1e-2
    layer = ca.ConcordLinearPackedB(768, 768, bias=True, device=DEV, lr=5e-4)
    flags = O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH
    if winner:
        pb.set_ratio_coh(True)
        pb.set_ratio_coh_floors(0.9, 0.999)
        layer.disable_cohpre()
        layer.gf_consol = 50.0
        flags |= O.RATIO_COH | O.GF_CONSOLIDATION
    else:
        flags |= O.COHPRE
    layer.load_weights(W0)
    p0, r0, c0 = O.load_weights(W0.numpy())
    np.testing.assert_array_equal(host(layer.packed_w), p0)
    state = [p0.copy(), r0.copy(), c0.copy(), np.zeros(768, np.float32), np.zeros(768, np.float32)]
    coh = None if winner else np.ones((768, 768), np.float32)
    for step in range(3):
        salt_next = int(host(pb._get_step_counter(DEV))[0]) + 1
        xd = x.to(DEV).requires_grad_(True)
        cap = []
        pb._DEBUG_CAPTURE = cap
        try:
            y = layer(xd)
            y.backward(gy.to(DEV))
        finally:
            pb._DEBUG_CAPTURE = None
        layer.rebalance()
        sync()
        rm, cm = _oracle_step(O, state, host(cap[0]), 5e-4, salt_next, flags, coh,
                              gf_consol=50.0 if winner else 0.0)
        O.rebalance(state[0], state[1], state[2], rm, cm, seed=step + 1)
        np.testing.assert_array_equal(host(layer.packed_w), state[0])
        np.testing.assert_array_equal(host(layer.row_exp), state[1])
        np.testing.assert_array_equal(host(layer.v_row), state[3])
        np.testing.assert_array_equal(host(layer.v_col), state[4])
    np.testing.assert_array_equal(host(layer.consolidated_weight()),
                                  O.materialize(state[0], state[1], state[2], consolidated=True))
    np.testing.assert_array_equal(host(layer.get_weight()), O.materialize(state[0], state[1], state[2]))


def test_layer_weight_cache_mode_matches_fused():
    """The two forward modes feed identical bf16 operands: same y, dx, state."""
    import concord_amd as ca
    torch.manual_seed(3)
    W0 = torch.randn(384, 256) * 0.05
    x = torch.randn(512, 256)
    gy = torch.randn(512, 384) * 1e-2
    outs = []
    from concord_amd import packed_b as pb
    for cache in (False, True):
        pb._get_step_counter(DEV).fill_(100)
        layer = ca.ConcordLinearPackedB(256, 384, bias=True, device=DEV, lr=1e-3, weight_cache=cache)
        layer.load_weights(W0)
        xd = x.to(DEV).requires_grad_(True)
        y = layer(xd)
        y.backward(gy.to(DEV))
        y2 = layer(xd.detach())
        sync()
        outs.append((host(y.to(torch.bfloat16)), host(xd.grad.to(torch.bfloat16)), host(layer.packed_w),
                     host(y2.to(torch.bfloat16))))
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)


def test_determinism_run_twice():
    import concord_amd as ca
    from concord_amd import packed_b as pb
    res = []
    for _ in range(2):
        torch.manual_seed(9)
        pb._get_step_counter(DEV).fill_(0)
        layer = ca.ConcordLinearPackedB(640, 320, bias=False, device=DEV, lr=2e-3)
        for _ in range(3):
            x = torch.randn(300, 640, device=DEV).requires_grad_(True)
            layer(x).square().mean().backward()
            layer.rebalance()
        sync()
        res.append(host(layer.packed_w))
    np.testing.assert_array_equal(res[0], res[1])


def test_bare_default_trains():
    """concord/test_baked_defaults.py:34-46: a bare layer fits a toy regression."""
    import concord_amd as ca
    torch.manual_seed(1)
    W = ca.ConcordLinearPackedB(32, 32, bias=False, device=DEV)
    W.lr = 0.02
    tgt = torch.randn(32, 32, device=DEV) * 0.3
    x = torch.randn(256, 32, device=DEV)
    y = x @ tgt.T
    losses = []
    for _ in range(80):
        xb = x.detach().requires_grad_(True)
        loss = torch.nn.functional.mse_loss(W(xb).float(), y)
        loss.backward()
        W.rebalance()
        losses.append(loss.item())
    assert losses[-1] < 0.9 * losses[0]
    W.disable_cohpre()
    assert W._coh_pre is None
    loss = torch.nn.functional.mse_loss(W(x.requires_grad_(True)).float(), y)
    loss.backward()
    W.rebalance()


def test_3d_input_and_fp32_dtype():
    import concord_amd as ca
    torch.manual_seed(2)
    layer = ca.ConcordLinearPackedB(96, 48, bias=True, device=DEV)
    x = torch.randn(4, 25, 96, device=DEV, requires_grad=True)
    y = layer(x)
    assert y.shape == (4, 25, 48) and y.dtype == torch.float32
    y.sum().backward()
    assert x.grad.shape == x.shape and layer.bias.grad is not None


# ---------------------------------------------------------------- Muon drive

@pytest.mark.parametrize("N,K", [(96, 160), (160, 96), (256, 1024), (1024, 256), (200, 333), (1, 8)])
def test_muon_ns5_matches_oracle(oracle, N, K):
    """O = gamma NS5(g / ||g||) on the GPU (bf16 MFMA products) against the
    oracle's bf16 restatement.  Tolerance 2e-2 rel-L2: the chain has 15 bf16
    products and 10 bf16 roundings, and two restatements of the same bf16
    method already differ by up to ~7e-3 where the accumulation order flips
    a rounding (tests/test_oracle_math.py)."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N * 3 + K)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 1e-3).astype(np.float32))
    gamma = float(np.float32(np.sqrt(np.float32(max(N, K)))))
    o = pb.muon_ns5(dev(g), gamma=gamma)
    sync()
    ref = oracle.bf16_bits_to_f32(oracle.muon_ns5(g, gamma)).astype(np.float64)
    got = oracle.bf16_bits_to_f32(host(o)).astype(np.float64)
    assert rel_l2(got, ref) < 2e-2


@pytest.mark.parametrize("M,R,b_rows", [(1280, 5120, 1), (1280, 1280, 0), (96, 160, 1), (200, 200, 0),
                                         (1000, 3000, 1)])
def test_gemm_bf16_sym_matches_float64(oracle, M, R, b_rows):
    """The symmetric product (only the tiles meeting the upper triangle, the
    rest mirrored): exactly symmetric; elementwise within one bf16 rounding
    plus the worst-case fp32 summation error of R terms (R 2^-24 sum |terms|)
    of the float64 product, and within 4e-3 rel-L2 of it (one bf16 rounding
    is ~1e-3)."""
    from concord_amd import _lib as C
    rng = np.random.default_rng(M + R + b_rows)
    a = oracle.f32_to_bf16_bits_array(rng.standard_normal((M, R)).astype(np.float32))
    af = oracle.bf16_bits_to_f32(a).astype(np.float64)
    if b_rows:
        b, exact, mag = a, af @ af.T, np.abs(af) @ np.abs(af).T
    else:   # a symmetric operand times itself
        s = (af + af.T) / 2
        a = oracle.f32_to_bf16_bits_array(s.astype(np.float32))
        af = oracle.bf16_bits_to_f32(a).astype(np.float64)
        b, exact, mag = a, af @ af, np.abs(af) @ np.abs(af)
    ad, bd = dev(a).view(torch.bfloat16), dev(b).view(torch.bfloat16)
    c = torch.empty((M, M), dtype=torch.bfloat16, device=DEV)
    ws = torch.zeros(int(C.lib().concord_gemm_sym_workspace_bytes(M, R, b_rows)), dtype=torch.uint8, device=DEV)
    C.check(C.lib().concord_gemm_bf16_sym(C.ptr(ad), R, C.ptr(bd), R if b_rows else M, b_rows, C.ptr(c), M, M, R,
                                          C.ptr(ws), ws.numel(), C.stream_of(torch.device(DEV))), "gemm_bf16_sym")
    sync()
    got = host(c).view(np.uint16)
    np.testing.assert_array_equal(got, got.T)
    g = oracle.bf16_bits_to_f32(got).astype(np.float64)
    tol = 2.0 ** -8 * np.abs(exact) + R * 2.0 ** -24 * mag
    assert np.all(np.abs(g - exact) <= tol), np.max(np.abs(g - exact) - tol)
    assert rel_l2(g, exact) < 4e-3


@pytest.mark.parametrize("N,K", [(1280, 5120), (5120, 1280)])
def test_muon_ns5_fused_combines_match_two_step(oracle, N, K):
    """NS5's two combinations ride in the epilogue of the product before them
    (A A -> B = bf16(b A + c bf16(A A)), B X -> X = bf16(a X + bf16(B X))).
    Re-running the two-step route -- the library's own bf16 GEMM entries
    (same tile and split plans: the symmetric product for X X^T and A A),
    the combinations in float32 on the host -- gives the same bits."""
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + 7)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 1e-3).astype(np.float32))
    gamma = float(np.float32(np.sqrt(np.float32(max(N, K)))))
    o = pb.muon_ns5(dev(g), gamma=gamma)
    sync()
    f32, bf = np.float32, oracle.f32_to_bf16_bits_array
    nrm = f32(np.sqrt(oracle.frob_sumsq(g)))
    den = f32(max(nrm, f32(1e-12)) * f32(f32(nrm / max(nrm, f32(1e-12))) + f32(1e-7)))
    gf = oracle.bf16_bits_to_f32(g)
    if N > K:
        gf = np.ascontiguousarray(gf.T)
    m, n = gf.shape
    X = bf((gf / den).astype(np.float32))
    ws = torch.zeros(int(C.lib().concord_muon_workspace_bytes(N, K)), dtype=torch.uint8, device=DEV)
    st = C.stream_of(torch.device(DEV))
    a, b, c = f32(3.4445), f32(-4.7750), f32(2.0315)
    for _ in range(5):
        Xd = dev(X).view(torch.bfloat16)
        A = torch.empty((m, m), dtype=torch.bfloat16, device=DEV)
        C.check(C.lib().concord_gemm_bf16_sym(C.ptr(Xd), n, C.ptr(Xd), n, 1, C.ptr(A), m, m, n,
                                              C.ptr(ws), ws.numel(), st), "X X^T")
        AA = torch.empty((m, m), dtype=torch.bfloat16, device=DEV)
        C.check(C.lib().concord_gemm_bf16_sym(C.ptr(A), m, C.ptr(A), m, 0, C.ptr(AA), m, m, m,
                                              C.ptr(ws), ws.numel(), st), "A A")
        sync()
        Af = oracle.bf16_bits_to_f32(host(A).view(np.uint16))
        AAf = oracle.bf16_bits_to_f32(host(AA).view(np.uint16))
        np.testing.assert_array_equal(host(A), host(A).T)     # mirrored: exactly symmetric
        np.testing.assert_array_equal(host(AA), host(AA).T)
        B = bf((b * Af + c * AAf).astype(np.float32))
        Bd = dev(B).view(torch.bfloat16)
        BX = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
        C.check(C.lib().concord_gemm_bf16_dgrad(C.ptr(Bd), m, C.ptr(Xd), n, C.ptr(BX), n, m, m, n,
                                                C.ptr(ws), ws.numel(), st), "B X")
        sync()
        BXf = oracle.bf16_bits_to_f32(host(BX).view(np.uint16))
        X = bf((a * oracle.bf16_bits_to_f32(X) + BXf).astype(np.float32))
    out = bf((f32(gamma) * oracle.bf16_bits_to_f32(X)).astype(np.float32))
    if N > K:
        out = np.ascontiguousarray(out.T)
    np.testing.assert_array_equal(host(o).view(np.uint16), out)


@pytest.mark.parametrize("N,K", [(2048, 5120), (1280, 5120), (333, 1001)])
def test_muon_frobenius_denominator_bit_exact(oracle, N, K):
    """The NS5 input scale n (||g|| / n + 1e-7), n = max(||g||, 1e-12) (block partials,
    then one wave: 64 lanes of ascending partial sums and a tree) equals the oracle's bit
    for bit; read back from the workspace (layout: the split-K region, X, BX,
    A, AA, partials, then the denominator in the last 256-byte slot)."""
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + K)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, K)) * 1e-3).astype(np.float32))
    gd = dev(g)
    pb.muon_ns5(gd)
    sync()
    ws = pb._MUON_WORKSPACES[pb._dev_key(torch.device(DEV))]
    off = int(C.lib().concord_muon_workspace_bytes(N, K)) - 256
    den = host(ws[off:off + 4].view(torch.float32))[0]
    s = oracle.frob_sumsq(g)
    nrm = np.float32(np.sqrt(np.float32(s)))
    n = max(nrm, np.float32(1e-12))
    want = np.float32(n * np.float32(np.float32(nrm / n) + np.float32(1e-7)))
    assert den.view(np.uint32) == np.float32(want).view(np.uint32), (den, want)


def test_muon_ns5_full_size_properties(oracle):
    """Config 5 shape (1280 x 5120): the drive's singular values lie in the
    quintic's band times gamma, a power-of-two rescale of g leaves the drive
    bit-identical, and two calls agree bit for bit (fixed reduction order)."""
    from concord_amd import packed_b as pb
    N, K = 1280, 5120
    g = torch.randn(N, K, generator=torch.Generator().manual_seed(3)) * 1e-3
    gd = g.to(torch.bfloat16).to(DEV)
    o1 = pb.muon_ns5(gd)
    o2 = pb.muon_ns5(gd)
    o4 = pb.muon_ns5((gd.float() * 4.0).to(torch.bfloat16))
    sync()
    a1 = host(o1)
    np.testing.assert_array_equal(a1, host(o2))
    np.testing.assert_array_equal(a1, host(o4))
    X = oracle.bf16_bits_to_f32(a1).astype(np.float64) / np.sqrt(K)
    ev = np.linalg.eigvalsh(X @ X.T)
    sv = np.sqrt(np.clip(ev, 0, None))
    assert sv.min() > 0.6 and sv.max() < 1.25, (sv.min(), sv.max())


def test_layer_muon_drive_bit_exact(oracle):
    """drive='muon': the backward feeds O = sqrt(max(N,K)) NS5(grad_W) to the
    update as its step (CONCORD_MUON: no v-hat, eps or cap); packed words and
    exponents bit-exact vs the oracle's update fed the same O."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    O = oracle
    N, K, M = 384, 256, 512
    torch.manual_seed(1)
    W0 = torch.nn.init.kaiming_uniform_(torch.empty(N, K), a=5 ** 0.5)
    x = torch.randn(M, K)
    gy = torch.randn(M, N) * 1e-2
    layer = ca.ConcordLinearPackedB(K, N, bias=False, device=DEV, lr=1e-3, drive='muon')
    pb.set_ratio_coh(True)
    pb.set_ratio_coh_floors(0.9, 0.999)
    try:
        layer.disable_cohpre()
        layer.gf_consol = 10.0
        layer.load_weights(W0)
        p0, r0, c0 = O.load_weights(W0.numpy())
        pk, re, ce = p0.copy(), r0.copy(), c0.copy()
        flags = (O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION | O.FIXED_COH
                 | O.RATIO_COH | O.GF_CONSOLIDATION | O.MUON)
        for step in range(3):
            salt_next = int(host(pb._get_step_counter(DEV))[0]) + 1
            cap = []
            pb._DEBUG_CAPTURE = cap
            try:
                y = layer(x.to(DEV).requires_grad_(True))
                y.backward(gy.to(DEV))
            finally:
                pb._DEBUG_CAPTURE = None
            layer.rebalance()
            sync()
            drive = host(cap[0])
            rm = np.zeros(N, np.int32)
            cm = np.zeros(K, np.int32)
            P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0,
                               precond_p=0.5, gf_consol=10.0, drift_cancel_C=0.018036072144288578,
                               alpha_v_fast=0.001, wd_sv=0.0, wd_sf=0.0, gf_trust_delta_sq=1.0,
                               gate_gain=1.0, mantissa_bias=15)
            S = O.UpdateScalars(lr=1e-3, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0,
                                salt=salt_next, consolidate=1)
            z = np.zeros(1, np.float32)
            O.apply_adamw(pk, drive, None, re, ce, rm, cm, np.zeros(N, np.float32), np.zeros(K, np.float32),
                          z[0], None, P, S, flags)
            O.rebalance(pk, re, ce, rm, cm, seed=step + 1)
            np.testing.assert_array_equal(host(layer.packed_w), pk)
            np.testing.assert_array_equal(host(layer.row_exp), re)
            # the drive is the NS5 of this step's gradient: unit-RMS scale, gamma-sized
            dv = O.bf16_bits_to_f32(drive).astype(np.float64)
            assert 0.4 < np.sqrt((dv * dv).mean()) < 1.2
    finally:
        pb.set_ratio_coh(False)


def _layer_state(layer):
    return [host(t) for t in (layer.packed_w, layer.row_exp, layer.col_exp, layer.v_row, layer.v_col,
                              layer._sum_v_inv, layer._row_max_buf, layer._col_max_buf, layer._reb_seed)]


def test_steps_reuse_buffers():
    """Steady-state steps allocate no new layer state: the packed words,
    exponents, v-hat state, watermark buffers and the per-device workspaces
    keep their storage from the second step on (the reference checks the
    same for its watermark buffers, notebook/src/test_prealloc_buffers.py:107-120)."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(21)
    layer = ca.ConcordLinearPackedB(256, 384, bias=True, device=DEV, lr=1e-3)
    x = torch.randn(512, 256, device=DEV)
    gy = torch.randn(512, 384, device=DEV) * 1e-2

    def step():
        layer(x.clone().requires_grad_(True)).backward(gy)
        layer.rebalance()

    def ptrs():
        names = ("packed_w", "row_exp", "col_exp", "v_row", "v_col", "_sum_v_inv", "_row_max_buf",
                 "_col_max_buf")
        out = {n: getattr(layer, n).data_ptr() for n in names}
        key = pb._dev_key(torch.device(DEV))
        out["ws"] = pb._WORKSPACES[key].data_ptr()
        out["gemm_ws"] = pb._GEMM_WORKSPACES[key].data_ptr()
        return out

    step()
    first = ptrs()
    for _ in range(3):
        step()
    sync()
    assert ptrs() == first


@pytest.mark.parametrize("M", [512, 154])
def test_graph_replay_matches_eager_steps(M):
    """A HIP graph of one training step (forward, backward with the update,
    rebalance), replayed with eager work and host syncs between replays,
    tracks an eager twin bit for bit on every replay.  At M = 154 the
    backward's products run in one launch and the finalize's launch carries
    the dgrad's split-K reduction (its ticket re-arms itself in the graph)."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(12)
    W0 = torch.randn(1280, 1280) * 0.03
    x = torch.randn(M, 1280, device=DEV).to(torch.bfloat16).requires_grad_(True)
    dy = (torch.randn(M, 1280, device=DEV) * 1e-3).to(torch.bfloat16)
    xe = x.detach().clone().requires_grad_(True)
    salt = pb._get_step_counter(DEV)

    def make():
        layer = ca.ConcordLinearPackedB(1280, 1280, bias=True, device=DEV, lr=2e-3)
        layer.load_weights(W0)
        return layer

    def step(layer, xin):
        xin.grad = None
        layer.bias.grad = None
        layer(xin).backward(dy)
        layer.rebalance()

    g_layer, e_layer = make(), make()
    # the graph layer's warm-up runs on a side stream, as capture requires
    salt.fill_(7)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step(g_layer, x)
    torch.cuda.current_stream().wait_stream(s)
    sync()
    salt.fill_(7)
    for _ in range(2):
        step(e_layer, xe)
    sync()
    for a, b in zip(_layer_state(g_layer), _layer_state(e_layer)):
        np.testing.assert_array_equal(a, b)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(g_layer, x)
    for r in range(4):
        salt.fill_(100 + r)
        graph.replay()
        sync()
        salt.fill_(100 + r)
        step(e_layer, xe)
        sync()
        for a, b in zip(_layer_state(g_layer) + [host(x.grad), host(g_layer.bias.grad)],
                        _layer_state(e_layer) + [host(xe.grad), host(e_layer.bias.grad)]):
            np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("cohpre", [True, False])
def test_checkpoint_resume_bit_exact(cohpre):
    """state_dict -> torch.save -> torch.load(weights_only=True) -> a fresh
    layer resumes bit for bit: packed words, exponents, v-hat, watermarks,
    coh_pre and the SR salt counter all travel (the reference loses the salt
    and coh_pre)."""
    import io
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(21)
    W0 = torch.randn(384, 256) * 0.05
    xs = [torch.randn(512, 256, device=DEV) for _ in range(5)]
    salt = pb._get_step_counter(DEV)
    salt.fill_(1234)

    def steps(layer, batch):
        for x in batch:
            xd = x.clone().requires_grad_(True)
            layer(xd).square().mean().backward()
            layer.rebalance()

    a = ca.ConcordLinearPackedB(256, 384, bias=True, device=DEV, lr=3e-3)
    if not cohpre:
        a.disable_cohpre()
        a.gf_consol = 20.0
    a.load_weights(W0)
    a.lr = 4e-3
    steps(a, xs[:3])
    buf = io.BytesIO()
    torch.save(a.state_dict(), buf)
    steps(a, xs[3:])
    sync()
    want = _layer_state(a) + [host(a.bias)]
    if cohpre:
        want.append(host(a._coh_pre))

    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    b = ca.ConcordLinearPackedB(256, 384, bias=True, device=DEV, lr=1e-1)
    salt.fill_(0)
    b.load_state_dict(sd)
    assert b.lr == pytest.approx(4e-3) and b.gf_consol == a.gf_consol
    assert (b._coh_pre is None) == (not cohpre)
    steps(b, xs[3:])
    sync()
    got = _layer_state(b) + [host(b.bias)]
    if cohpre:
        got.append(host(b._coh_pre))
    for u, v in zip(want, got):
        np.testing.assert_array_equal(u, v)


# the reference class's state_dict keys: its registered buffers and the bias
# parameter (concord/packed_b.py:1445-1492)
REFERENCE_KEYS = ['_reb_seed', 'packed_w', 'row_exp', 'col_exp', 'v_row', 'v_col', '_sum_v_inv',
                  '_row_max_hwm', '_col_max_hwm', '_lr_buf', '_eps_buf', 'bias']


class _ReferenceShaped(torch.nn.Module):
    """A module with exactly the reference class's buffers and parameter."""

    def __init__(self, N, K, bias=True):
        super().__init__()
        z = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt, device=DEV)  # noqa: E731
        self.register_buffer('_reb_seed', z(1, dt=torch.int32))
        self.register_buffer('packed_w', z(N, K, dt=torch.int32))
        self.register_buffer('row_exp', z(N, dt=torch.int8))
        self.register_buffer('col_exp', z(K, dt=torch.int8))
        self.register_buffer('v_row', z(N))
        self.register_buffer('v_col', z(K))
        self.register_buffer('_sum_v_inv', z(1))
        self.register_buffer('_row_max_hwm', z(N, dt=torch.int32))
        self.register_buffer('_col_max_hwm', z(K, dt=torch.int32))
        self.register_buffer('_lr_buf', z(1))
        self.register_buffer('_eps_buf', z(1))
        self.bias = torch.nn.Parameter(z(N, dt=torch.bfloat16)) if bias else None


def test_state_dict_interchanges_with_reference_key_set():
    """Checkpoints cross between this class and the reference's in both
    directions under strict loading: a state_dict with only the reference's
    keys loads here (the salt counter and coh_pre keep their values, lr / eps
    follow the loaded device scalars), and reference_state_dict() strips the
    extra-state entry so the result loads into a module with the
    reference's buffers."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(23)
    a = ca.ConcordLinearPackedB(96, 64, bias=True, device=DEV, lr=2e-3)
    x = torch.randn(128, 96, device=DEV).requires_grad_(True)
    a(x).square().mean().backward()
    a.rebalance()
    a.lr = 7e-4
    sd = ca.reference_state_dict(a)
    assert sorted(sd) == sorted(REFERENCE_KEYS)
    assert '_extra_state' in a.state_dict()
    # this build -> the reference's key set
    r = _ReferenceShaped(64, 96)
    r.load_state_dict(sd, strict=True)
    np.testing.assert_array_equal(host(r.packed_w), host(a.packed_w))
    # the reference's key set -> this build
    salt = pb._get_step_counter(DEV)
    salt.fill_(555)
    b = ca.ConcordLinearPackedB(96, 64, bias=True, device=DEV, lr=1e-1)
    cp = b._coh_pre
    res = b.load_state_dict(r.state_dict(), strict=True)
    assert not res.missing_keys and not res.unexpected_keys
    sync()
    for k in REFERENCE_KEYS:
        np.testing.assert_array_equal(host(getattr(b, k)), host(getattr(a, k)))
    assert b.lr == pytest.approx(7e-4) and int(host(salt)[0]) == 555 and b._coh_pre is cp
    # a checkpoint of this build still needs its extra state under strict
    # loading only through the key it wrote: a foreign key still fails
    with pytest.raises(RuntimeError):
        b.load_state_dict(dict(sd, stray=torch.zeros(1)), strict=True)


def test_consolidated_state_dict_matches_layers():
    import concord_amd as ca
    torch.manual_seed(22)
    layers = [ca.ConcordLinearPackedB(128, 64, bias=True, device=DEV),
              ca.ConcordLinearPackedB(64, 32, bias=False, device=DEV)]
    sd = ca.consolidated_state_dict(layers, ["a", "b"])
    assert set(sd) == {"a.weight", "a.bias", "b.weight"}
    np.testing.assert_array_equal(host(sd["a.weight"]), host(layers[0].consolidated_weight()))
    np.testing.assert_array_equal(host(sd["b.weight"]), host(layers[1].consolidated_weight()))
    assert sd["a.weight"].dtype == torch.bfloat16 and sd["a.weight"].shape == (64, 128)


# ---------------------------------------------------------------- multi-layer statistics

# (4096, 2112): 1056 block partials, so the final chain takes two staging rounds of up to 1024
@pytest.mark.parametrize("N,K,ld", [(300, 777, 777), (5120, 1280, 1280), (33, 100, 128), (1, 5, 5),
                                    (4096, 2112, 2112)])
def test_coherence_sum_bit_exact(oracle, N, K, ld):
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + K)
    words = rng.integers(-2 ** 31, 2 ** 31, (N, ld), dtype=np.int64).astype(np.int32)
    Cc = 0.018036072144288578
    p = dev(words)
    out = torch.empty(1, dtype=torch.float32, device=DEV)
    ws = pb._stats_workspace(torch.device(DEV), 0, N * K)
    assert C.lib().concord_coherence_sum(C.ptr(p), ld, N, K, Cc, C.ptr(out), C.ptr(ws), ws.numel(),
                                         C.stream_of(torch.device(DEV))) == 0
    sync()
    want = oracle.coherence_sum(np.ascontiguousarray(words[:, :K]), Cc)
    assert host(out)[0].view(np.uint32) == np.float32(want).view(np.uint32)


def test_measure_coherence_layer(oracle):
    import concord_amd as ca
    torch.manual_seed(5)
    layer = ca.ConcordLinearPackedB(256, 384, device=DEV)
    x = torch.randn(512, 256, device=DEV).requires_grad_(True)
    for _ in range(3):
        layer(x).square().mean().backward()
    sync()
    got = ca.measure_coherence(layer)
    want = float(oracle.coherence_sum(host(layer.packed_w), layer.drift_cancel_C)) / (256 * 384)
    assert got == want and 0.0 <= got <= 1.0


@pytest.mark.parametrize("nr,nc", [(0, 0), (7, 0), (0, 9), (5000, 70000), (123457, 3)])
def test_watermark_peak(nr, nc):
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(nr * 7 + nc)
    r = rng.integers(0, 30000, max(nr, 1)).astype(np.int32)[:nr]
    c = rng.integers(0, 30000, max(nc, 1)).astype(np.int32)[:nc]
    rd, cd = dev(r) if nr else torch.zeros(1, dtype=torch.int32, device=DEV), \
        dev(c) if nc else torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.full((1,), -5, dtype=torch.int32, device=DEV)
    ws = pb._stats_workspace(torch.device(DEV), nr + nc, 0)
    assert C.lib().concord_watermark_peak(C.ptr(rd), nr, C.ptr(cd), nc, C.ptr(out), C.ptr(ws), ws.numel(),
                                          C.stream_of(torch.device(DEV))) == 0
    sync()
    want = max([0] + ([int(r.max())] if nr else []) + ([int(c.max())] if nc else []))
    assert int(host(out)[0]) == want


@pytest.mark.parametrize("device_gate", [True, False])
def test_gated_rebalance_matches_host_gate(device_gate):
    """GatedRebalance (shared watermark slabs, one device reduction, the
    comparison with MAX_M on the device or on the host) takes the same
    decisions and leaves every layer bit-identical to the same gate
    evaluated on the host (max of every layer's watermarks > MAX_M, then the
    per-layer rebalance loop), over several training steps."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    shapes = [(256, 384), (384, 128), (128, 256)]   # (in, out), chained
    torch.manual_seed(31)
    Ws = [torch.randn(n, k) / k ** 0.5 for k, n in shapes]
    xs = [torch.randn(300, shapes[0][0], device=DEV) for _ in range(4)]
    salt = pb._get_step_counter(DEV)
    results, decisions = [], []
    for gated in (True, False):
        layers = [ca.ConcordLinearPackedB(k, n, bias=False, device=DEV, lr=5e-3) for k, n in shapes]
        for m, W in zip(layers, Ws):
            m.load_weights(W)
        gate = ca.GatedRebalance(layers, device_gate=device_gate)
        fired = []
        for i, x in enumerate(xs):
            salt.fill_(70 + i)
            h = x.clone().requires_grad_(True)
            for m in layers:
                h = m(h)
            h.square().mean().backward()
            if gated:
                before = gate.fires
                gate()
                fired.append(gate.fires > before)
            elif i == 0:
                fired.append(False)   # the gate's first call only wires the slabs
            else:
                peak = max(int(t.max().item()) for m in layers for t in (m._row_max_buf, m._col_max_buf))
                fired.append(peak > m.MAX_M)
                if fired[-1]:
                    for m in layers:
                        m.rebalance()
        sync()
        decisions.append(fired)
        results.append([host(t) for m in layers for t in (m.packed_w, m.row_exp, m.col_exp, m._reb_seed)])
    assert decisions[0] == decisions[1]
    for a, b in zip(*results):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("device_gate", [True, False])
def test_gated_rebalance_gate_logic(device_gate):
    """Below MAX_M nothing runs (no seed advance); one watermark above it
    fires the rebalance of every layer."""
    import concord_amd as ca
    layers = [ca.ConcordLinearPackedB(64, 96, bias=False, device=DEV),
              ca.ConcordLinearPackedB(96, 32, bias=False, device=DEV)]
    gate = ca.GatedRebalance(layers, device_gate=device_gate)
    assert gate() is False and gate.row_all is not None
    seeds = [int(host(m._reb_seed)[0]) for m in layers]
    gate.row_all.fill_(gate.MAX_M)
    gate.col_all.fill_(7)
    assert gate() is (None if device_gate else False)
    assert [int(host(m._reb_seed)[0]) for m in layers] == seeds
    assert gate.fires == 0
    gate.col_all[40] = gate.MAX_M + 1
    assert gate() is (None if device_gate else True)
    assert gate.fires == 1
    assert [int(host(m._reb_seed)[0]) for m in layers] == [v + 1 for v in seeds]


@pytest.mark.parametrize("gain", [0.0, 0.37, 0.999])
def test_materialize_gated_bit_exact(oracle, gain):
    from concord_amd import _lib as C
    rng = np.random.default_rng(int(gain * 1000))
    N, K = 97, 1030
    packed = rng.integers(-2 ** 31, 2 ** 31, (N, K), dtype=np.int64).astype(np.int32)
    re = rng.integers(-8, 8, N).astype(np.int8)
    ce = rng.integers(-8, 8, K).astype(np.int8)
    out = torch.empty((N, K), dtype=torch.bfloat16, device=DEV)
    # the device copies stay referenced until the kernel has run
    pd, red, ced = dev(packed), dev(re), dev(ce)
    assert C.lib().concord_materialize_gated(C.ptr(pd), K, C.ptr(red), C.ptr(ced), N, K, 15, gain, C.ptr(out), K,
                                             C.stream_of(torch.device(DEV))) == 0
    sync()
    np.testing.assert_array_equal(host(out).view(np.uint16), oracle.materialize_gated(packed, re, ce, gain))


def test_layer_fast_gain_forward(oracle):
    """fast_gain < 1: the forward multiplies by the gated weight (within the
    GEMM tolerance of an fp32 product with the oracle's gated weight)."""
    import concord_amd as ca
    torch.manual_seed(8)
    layer = ca.ConcordLinearPackedB(256, 192, bias=False, device=DEV)
    layer.fast_gain = 0.25
    x = torch.randn(300, 256, device=DEV)
    y = layer(x)
    sync()
    Wg = oracle.bf16_bits_to_f32(oracle.materialize_gated(host(layer.packed_w), host(layer.row_exp),
                                                          host(layer.col_exp), 0.25)).astype(np.float64)
    ref = host(x.to(torch.bfloat16).float()).astype(np.float64) @ Wg.T
    assert rel_l2(host(y.float()).astype(np.float64), ref) < 1e-2


@pytest.mark.parametrize("M,N,K", [(2048, 5120, 1280), (2048, 1280, 1280), (4096, 1280, 1280), (1024, 2560, 640),
                                   (300, 384, 256), (154, 1280, 2048), (308, 1280, 2048), (308, 640, 2048),
                                   (4, 1280, 2816), (77, 320, 1280), (64, 64, 256), (40, 72, 200)])
def test_dgrad_wgrad_vhat_matches_separate_calls(M, N, K):
    """The combined backward entry gives the same dx, grad_W, bias gradient,
    v-hat state, zeroed watermarks and salt as the two calls.  Where the shapes
    allow, one launch carries the other's split-K reduction: the WGRAD launch
    the dgrad's (2048 x 5120 x 1280), or the unsplit dgrad launch the split
    WGRAD's v-hat reduction (4096 x 1280 x 1280, config 4's attention layers).
    For a few hundred tokens (cross-attention at 154 and 308, the M = 4
    embedding layers, a ragged 77) both products run in one launch
    (gemm_dgt_tr_kernel), the dgrad's split-K reduction after it; at 64 x 64 x
    256 the dgrad is unsplit in that launch, at 40 x 72 x 200 the edges are
    partial tiles."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N + K)
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-3, 3))
    pk, red, ced = dev(packed), dev(re), dev(ce)
    dy = (torch.randn(M, N, device=DEV) * 1e-2).to(torch.bfloat16)
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    outs = []
    for combined in (True, False):
        vr = torch.full((N,), 1e-4, device=DEV)
        vc = torch.full((K,), 2e-4, device=DEV)
        svi = torch.ones(1, device=DEV)
        rm = torch.full((N,), 77, dtype=torch.int32, device=DEV)
        cm = torch.full((K,), 88, dtype=torch.int32, device=DEV)
        salt = torch.full((1,), 5, dtype=torch.int32, device=DEV)
        if combined:
            dx, gw, gb = pb._dgrad_wgrad_vhat(dy, x, pk, red, ced, 15, vr, vc, svi, 0.999, rm, cm, salt,
                                              with_bias=True)
        else:
            dx = pb._gemm_dgrad(dy, pk, red, ced, 15, None)
            gw, gb = pb._wgrad_vhat(dy, x, vr, vc, svi, 0.999, rm, cm, salt, with_bias=True)
        sync()
        outs.append([host(t) for t in (dx, gw, gb, vr, vc, svi, rm, cm, salt)])
    for a, b in zip(*outs):
        np.testing.assert_array_equal(a, b)
    assert (outs[0][6] == 0).all() and outs[0][8][0] == 6


def _update_backward(pb, combined, dy, x, st, winner, lr, fuse=1):
    """One backward step of the fused-forward layer with the adamw update:
    the combined entry (combined = True; fuse: whether it may carry the update
    in the WGRAD launch; returns whether it did) or the v-hat entry then the
    separate update."""
    import ctypes
    from concord_amd import _lib as C
    M, N = dy.shape
    K = x.shape[1]
    pk, red, ced, vr, vc, svi, rm, cm, cp = st
    dcc = pb.compute_drift_cancel_C(0.1, 0.001, mass_preserve=True)
    gf = 50.0 if winner else 0.0
    if not combined:
        dx, gw, gb = pb._dgrad_wgrad_vhat(dy, x, pk, red, ced, 15, vr, vc, svi, 0.999, rm, cm,
                                          pb._get_step_counter(DEV), with_bias=True)
        pb.apply_packed_adamw(pk, gw, None, red, ced, rm, cm, lr=lr, eps=1e-10, v_scale=0.0, gf_consol=gf,
                              drift_cancel_C=dcc, mass_preserve=True, v_row=vr, v_col=vc, sum_v_inv=svi,
                              gf_trust_delta_sq=1.0, coh_pre=cp, salt_prebumped=True)
        return dx, gw, gb, None
    flags, P, S = pb._adamw_setup(DEV, lr, 15, 0.1, 0.0, 0.0, 1e-10, 10.0, 0.0, 0.5, gf, dcc, 0.001, 0.0, 0.0,
                                  True, True, True, 1.0, cp, False, True, False)
    dx = torch.empty((M, K), dtype=torch.bfloat16, device=DEV)
    gw = torch.empty((N, K), dtype=torch.bfloat16, device=DEV)
    gb = torch.empty(N, dtype=torch.bfloat16, device=DEV)
    gws = pb._gemm_workspace(DEV, M, N, K)
    ws = pb._workspace(DEV, N, K, M)
    fused = ctypes.c_int(-1)
    C.check(C.lib().concord_dgrad_wgrad_update(
        C.ptr(dy), dy.stride(0), C.ptr(pk), pk.stride(0), C.ptr(red), C.ptr(ced), C.ptr(dx), dx.stride(0),
        C.ptr(x), x.stride(0), C.ptr(gw), gw.stride(0), 1, fuse, M, N, K, 0.999, C.ptr(vr), C.ptr(vc), C.ptr(svi),
        C.ptr(rm), C.ptr(cm), C.ptr(cp), cp.stride(0) if cp is not None else K, C.ptr(gb), ctypes.byref(P),
        ctypes.byref(S), flags, C.ptr(ws), ws.numel(), C.ptr(gws), gws.numel(), ctypes.byref(fused),
        C.stream_of(DEV)), "dgrad_wgrad_update")
    return dx, gw, gb, fused.value


@pytest.mark.parametrize("fuse", [1, 0])
@pytest.mark.parametrize("winner", [True, False])
@pytest.mark.parametrize("M,N,K", [(2048, 5120, 1280), (2048, 1280, 1280), (4096, 1280, 1280), (1024, 2560, 640),
                                   (300, 384, 256), (0, 320, 192), (154, 1280, 2048), (308, 640, 2048)])
def test_dgrad_wgrad_update_matches_two_pass(M, N, K, winner, fuse):
    """concord_dgrad_wgrad_update against concord_dgrad_wgrad_vhat followed by
    concord_apply_adamw, two steps in a row from the same state: dx, the
    grad_W copy, the bias gradient, v_row, v_col, 1 / sum v_row, the
    watermarks, the salt, the packed words and coh_pre all bit-identical.
    fuse = 1: at the north-star shape the combined launch must carry the
    update, and its grid barriers must not report a fault; fuse = 0: the
    separate launches, 1 / sum v_row formed in the update from the
    finalize's 256-row totals."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N + K + winner)
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-3, 3))
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    dys = [(torch.randn(M, N, device=DEV) * 1e-2).to(torch.bfloat16) for _ in range(2)]
    vr0 = dev((rng.random(N) * 1e-3 + 1e-7).astype(np.float32))
    vc0 = dev((rng.random(K) * 1e-3 + 1e-7).astype(np.float32))
    cp0 = None if winner else dev(rng.random((N, K)).astype(np.float32))
    pb.set_ratio_coh(winner)
    pb.set_ratio_coh_floors(0.9, 0.999)
    try:
        runs = []
        for combined in (True, False):
            pb._get_step_counter(DEV).fill_(11)
            st = [dev(packed.copy()), dev(re), dev(ce), vr0.clone(), vc0.clone(), torch.ones(1, device=DEV),
                  torch.full((N,), 77, dtype=torch.int32, device=DEV),
                  torch.full((K,), 88, dtype=torch.int32, device=DEV),
                  None if winner else cp0.clone()]
            out = []
            for dy in dys:
                dx, gw, gb, fused = _update_backward(pb, combined, dy, x, st, winner, 5e-4, fuse)
                sync()
                out.append(([host(t) for t in (dx, gw, gb)] + [host(t) for t in st if t is not None] +
                            [host(pb._get_step_counter(DEV))], fused))
            runs.append(out)
        for (a, fused), (b, _) in zip(*runs):
            if (M, N, K) == (2048, 5120, 1280) or not fuse:
                assert fused == fuse
            for u, v in zip(a, b):
                np.testing.assert_array_equal(u, v)
        assert not pb.wgrad_update_faults(DEV)
    finally:
        pb.set_ratio_coh(False)


def test_layer_fused_update_matches_separate():
    """The module's backward through the combined entry (set_fused_update)
    against the separate launches: 3 winner-flag steps of the north-star
    layer (1280 -> 5120, 2048 tokens, bias) with rebalance, same words,
    exponents, v-hat state, grad_x and bias gradient."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(4)
    W0 = torch.randn(5120, 1280) * 0.02
    xs = [torch.randn(2048, 1280, device=DEV) for _ in range(3)]
    gys = [torch.randn(2048, 5120, device=DEV) * 1e-2 for _ in range(3)]
    pb.set_ratio_coh(True)
    pb.set_ratio_coh_floors(0.9, 0.999)
    res = []
    try:
        for fused in (True, False):
            pb.set_fused_update(fused)
            pb._get_step_counter(DEV).fill_(3)
            layer = ca.ConcordLinearPackedB(1280, 5120, bias=True, device=DEV, lr=5e-4)
            layer.disable_cohpre()
            layer.gf_consol = 50.0
            layer.load_weights(W0)
            out = []
            for x, gy in zip(xs, gys):
                xd = x.clone().requires_grad_(True)
                layer.bias.grad = None
                layer(xd).backward(gy)
                layer.rebalance()
                sync()
                out += [host(xd.grad.to(torch.bfloat16)), host(layer.bias.grad.to(torch.bfloat16))]
            out += [host(t) for t in (layer.packed_w, layer.row_exp, layer.col_exp, layer.v_row, layer.v_col)]
            res.append(out)
        for a, b in zip(*res):
            np.testing.assert_array_equal(a, b)
        assert not pb.wgrad_update_faults(DEV)
    finally:
        pb.set_fused_update(False)
        pb.set_ratio_coh(False)


def test_fused_update_graph_replays_match_eager():
    """The layer step through the combined backward launch (set_fused_update)
    captured in a HIP graph and replayed three times, each replay followed by
    an eager step of a twin layer through the separate launches from the same
    state and salt: words, exponents, v-hat state and bias gradients identical
    after every replay (the launch re-arms its own barrier counters; no memset
    is recorded), and no barrier fault."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(6)
    W0 = torch.randn(5120, 1280) * 0.02
    x = torch.randn(2048, 1280, device=DEV)
    gy = torch.randn(2048, 5120, device=DEV) * 1e-2
    pb.set_ratio_coh(True)
    pb.set_ratio_coh_floors(0.9, 0.999)
    salt = pb._get_step_counter(DEV)
    layers = []
    for _ in range(2):
        la = ca.ConcordLinearPackedB(1280, 5120, bias=True, device=DEV, lr=5e-4)
        la.disable_cohpre()
        la.gf_consol = 50.0
        la.load_weights(W0)
        layers.append(la)
    xa = x.clone().requires_grad_(True)
    xb = x.clone().requires_grad_(True)

    def step(layer, xin):
        xin.grad = None
        layer.bias.grad = None
        layer(xin).backward(gy)
        layer.rebalance()

    def state(layer, xin):
        return [host(t) for t in (layer.packed_w, layer.row_exp, layer.col_exp, layer.v_row, layer.v_col,
                                  layer.bias.grad.to(torch.bfloat16), xin.grad.to(torch.bfloat16))]

    try:
        for k in range(2):   # eager warm-up of both twins, same salts
            salt.fill_(40 + k)
            pb.set_fused_update(True)
            step(layers[0], xa)
            salt.fill_(40 + k)
            pb.set_fused_update(False)
            step(layers[1], xb)
        sync()
        for u, v in zip(state(layers[0], xa), state(layers[1], xb)):
            np.testing.assert_array_equal(u, v)
        pb.set_fused_update(True)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                step(layers[0], xa)
        torch.cuda.current_stream().wait_stream(s)
        pb.set_fused_update(False)
        for k in range(3):
            salt.fill_(50 + k)
            g.replay()
            sync()
            assert int(host(salt)[0]) == 51 + k
            salt.fill_(50 + k)
            step(layers[1], xb)
            sync()
            for u, v in zip(state(layers[0], xa), state(layers[1], xb)):
                np.testing.assert_array_equal(u, v)
        assert not pb.wgrad_update_faults(DEV)
    finally:
        pb.set_fused_update(False)
        pb.set_ratio_coh(False)


@pytest.mark.parametrize("N,K", [(320, 192), (5120, 1280)])
def test_empty_batch_wgrad_entries(oracle, N, K):
    """M = 0 tokens: the weight gradient is the sum over no tokens, so the
    wgrad entries write zeros and the v-hat entries run the EMA of that zero
    gradient (v decays, watermarks zeroed, salt advanced, bias gradient 0).
    The empty activations may have NULL data pointers.  (At 5120 x 1280 the
    WGRAD tile rows exceed the operand, the case whose buffer size used to
    go negative.)"""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + K)
    packed, re, ce = rand_state(rng, N, K)
    pk, red, ced = dev(packed), dev(re), dev(ce)
    dy = torch.empty((0, N), dtype=torch.bfloat16, device=DEV)
    x = torch.empty((0, K), dtype=torch.bfloat16, device=DEV)
    gw = pb._wgrad(dy, x)
    sync()
    assert (host(gw) == 0).all()
    vr0 = (rng.random(N) * 1e-3 + 1e-7).astype(np.float32)
    vc0 = (rng.random(K) * 1e-3 + 1e-7).astype(np.float32)
    evr, evc = vr0.copy(), vc0.copy()
    esvi = oracle.vhat_ema(np.zeros((N, K), np.uint16), evr, evc, 0.999)
    for combined in (False, True):
        vr, vc = dev(vr0.copy()), dev(vc0.copy())
        svi = torch.ones(1, device=DEV)
        rm = torch.full((N,), 77, dtype=torch.int32, device=DEV)
        cm = torch.full((K,), 88, dtype=torch.int32, device=DEV)
        salt = torch.full((1,), 5, dtype=torch.int32, device=DEV)
        if combined:
            dx, gw, gb = pb._dgrad_wgrad_vhat(dy, x, pk, red, ced, 15, vr, vc, svi, 0.999, rm, cm, salt,
                                              with_bias=True)
            assert tuple(dx.shape) == (0, K)
        else:
            gw, gb = pb._wgrad_vhat(dy, x, vr, vc, svi, 0.999, rm, cm, salt, with_bias=True)
        sync()
        assert (host(gw) == 0).all() and (host(gb) == 0).all()
        np.testing.assert_array_equal(host(vr), evr)
        np.testing.assert_array_equal(host(vc), evc)
        assert host(svi)[0] == esvi
        assert (host(rm) == 0).all() and (host(cm) == 0).all() and host(salt)[0] == 6


def test_empty_batch_conv_wgrad_entries(oracle):
    """B = 0 images through the implicit conv's weight-gradient entries: a
    zero tap-major and packed-order gradient, and the v-hat EMA of zeros."""
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    geom = (0, 64, 16, 16, 320, 3, 3, 1, 1, 1, 1)
    B, Cin, H, W, Cout, kh, kw, sh, sw, ph, pw = geom
    K = Cin * kh * kw
    st = C.stream_of(DEV)
    gt = torch.full((Cout, K), 0x1234, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    ws = torch.zeros(int(C.lib().concord_conv_workspace_bytes(*geom)) + 4096, dtype=torch.uint8, device=DEV)
    C.check(C.lib().concord_conv_wgrad(None, None, C.ptr(gt), *geom, C.ptr(ws), ws.numel(), st), "conv_wgrad")
    sync()
    assert (host(gt) == 0).all()
    rng = np.random.default_rng(3)
    vr0 = (rng.random(Cout) * 1e-3 + 1e-7).astype(np.float32)
    vc0 = (rng.random(K) * 1e-3 + 1e-7).astype(np.float32)
    evr, evc = vr0.copy(), vc0.copy()
    esvi = oracle.vhat_ema(np.zeros((Cout, K), np.uint16), evr, evc, 0.999)
    gt.view(torch.int16).fill_(0x1234)
    gw = torch.full((Cout, K), 0x4321, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    gb = torch.full((Cout,), 0x1111, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    vr, vc = dev(vr0.copy()), dev(vc0.copy())
    svi = torch.ones(1, device=DEV)
    rm = torch.full((Cout,), 7, dtype=torch.int32, device=DEV)
    cm = torch.full((K,), 8, dtype=torch.int32, device=DEV)
    salt = torch.full((1,), 11, dtype=torch.int32, device=DEV)
    wsu = pb._workspace(DEV, Cout, K, 0)
    C.check(C.lib().concord_conv_wgrad_vhat(
        None, None, C.ptr(gt), C.ptr(gw), gw.stride(0), *geom, 0.999, C.ptr(vr), C.ptr(vc), C.ptr(svi),
        C.ptr(rm), C.ptr(cm), C.ptr(salt), C.ptr(gb), C.ptr(wsu), wsu.numel(), C.ptr(ws), ws.numel(), st),
        "conv_wgrad_vhat")
    sync()
    assert (host(gt) == 0).all() and (host(gw) == 0).all() and (host(gb) == 0).all()
    np.testing.assert_array_equal(host(vr), evr)
    np.testing.assert_array_equal(host(vc), evc)
    assert host(svi)[0] == esvi
    assert (host(rm) == 0).all() and (host(cm) == 0).all() and host(salt)[0] == 12


# ---------------------------------------------------------------- gradient noise

@pytest.mark.parametrize("N,K,ld,sigma", [(384, 256, 256, 0.1), (5120, 1280, 1280, 0.5), (33, 100, 104, 2.0)])
def test_iso_noise_bit_exact(oracle, N, K, ld, sigma):
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(N + K)
    g = oracle.f32_to_bf16_bits_array((rng.standard_normal((N, ld)) * 1e-3).astype(np.float32))
    gd = dev(g)
    salt = torch.full((1,), 4242, dtype=torch.int32, device=DEV)
    sig = torch.full((1,), sigma, dtype=torch.float32, device=DEV)
    pb.iso_noise_(gd[:, :K], sigma=sig, salt_counter=salt)
    sync()
    out = host(gd).view(np.uint16)
    np.testing.assert_array_equal(out[:, :K], oracle.iso_noise(np.ascontiguousarray(g[:, :K]), sigma, 4242))
    np.testing.assert_array_equal(out[:, K:], g[:, K:])   # the row padding is untouched
    assert int(host(salt)[0]) == 4242


def test_layer_iso_noise_step(oracle):
    """With the isotropic noise on, backward feeds the v-hat EMA and the
    update the noisy gradient: the captured grad_W equals the oracle's
    injection applied to the plain product, at the salt of the step."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(13)
    layer = ca.ConcordLinearPackedB(256, 384, bias=True, device=DEV, lr=1e-3)
    x = torch.randn(512, 256, device=DEV).to(torch.bfloat16)
    gy = (torch.randn(512, 384, device=DEV) * 1e-2).to(torch.bfloat16)
    salt = pb._get_step_counter(DEV)
    salt.fill_(900)
    ca.set_sigmag_noise(True, isotropic=True)
    ca.set_sigmag_sigma(0.2)
    cap = []
    pb._DEBUG_CAPTURE = cap
    try:
        xd = x.clone().requires_grad_(True)
        layer(xd).backward(gy)
    finally:
        pb._DEBUG_CAPTURE = None
        ca.set_sigmag_noise(False)
        ca.set_sigmag_sigma(0.0)
    sync()
    plain = host(pb._wgrad(gy, x)).view(np.uint16)
    want = oracle.iso_noise(plain, 0.2, 900)
    np.testing.assert_array_equal(host(cap[0]).view(np.uint16), want)
    assert int(host(salt)[0]) == 901 and layer.bias.grad is not None


def test_layer_muon_noise_is_post_ns(oracle):
    """drive='muon' with the noise on: NS5 runs on the clean gradient and the
    isotropic draw is added after it, scaled to sigma ||O||
    (docs/MUON_IMPLEMENTATION.md:21, 64-66), whichever draw was selected.
    The captured drive equals the oracle's injection applied to the GPU's
    NS5 of the plain product; at sigma = 0 the step is bit-identical to the
    step with the noise off."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(17)
    x = torch.randn(512, 256, device=DEV).to(torch.bfloat16)
    gy = (torch.randn(512, 384, device=DEV) * 1e-2).to(torch.bfloat16)
    salt = pb._get_step_counter(DEV)

    def run(noise, sigma, isotropic=False):
        torch.manual_seed(5)
        layer = ca.ConcordLinearPackedB(256, 384, bias=False, device=DEV, lr=1e-3, drive='muon')
        salt.fill_(700)
        ca.set_sigmag_noise(noise, isotropic=isotropic)
        ca.set_sigmag_sigma(sigma)
        cap = []
        pb._DEBUG_CAPTURE = cap
        try:
            layer(x.clone().requires_grad_(True)).backward(gy)
        finally:
            pb._DEBUG_CAPTURE = None
            ca.set_sigmag_noise(False)
            ca.set_sigmag_sigma(0.0)
        sync()
        return host(cap[0]).view(np.uint16), host(layer.packed_w)

    clean = host(pb.muon_ns5(pb._wgrad(gy, x))).view(np.uint16)
    for isotropic in (False, True):
        drive, _ = run(True, 0.3, isotropic)
        np.testing.assert_array_equal(drive, oracle.iso_noise(clean, 0.3, 700))
    d_off, p_off = run(False, 0.0)
    d_zero, p_zero = run(True, 0.0)
    np.testing.assert_array_equal(d_off, clean)
    np.testing.assert_array_equal(d_zero, clean)
    np.testing.assert_array_equal(p_zero, p_off)
    assert int(host(salt)[0]) == 701


@pytest.mark.parametrize("M,N,K", [(512, 384, 256), (2048, 1280, 640), (77, 96, 40)])
def test_sigmag_noise_parts(oracle, M, N, K):
    """The Sigma_g draw: the scaled dy and the token sum bit-exact against
    the oracle, the product (eps dy)^T x within 1e-2 of fp32, and the
    combine bit-exact against the oracle given that product (all read back
    from the workspace)."""
    from concord_amd import packed_b as pb
    rng = np.random.default_rng(M + N)
    dy = (torch.randn(M, N, device=DEV) * 1e-2).to(torch.bfloat16)
    x = torch.randn(M, K, device=DEV).to(torch.bfloat16)
    g0 = pb._wgrad(dy, x)
    g = g0.clone()
    salt = torch.full((1,), 313, dtype=torch.int32, device=DEV)
    sig = torch.full((1,), 0.3, dtype=torch.float32, device=DEV)
    pb.sigmag_noise_(g, dy, x, sigma=sig, salt_counter=salt)
    sync()
    ws = pb._SIGMAG_WORKSPACES[pb._dev_key(torch.device(DEV))]
    r256 = lambda b: (b + 255) // 256 * 256  # noqa: E731
    # layout: split-K region, scaled dy, product, partials, token partials,
    # sum, scale, draws (the split-K region's size is what the rest leaves)
    from concord_amd import _lib as C
    rest = (r256(M * N * 2) + r256(N * K * 2) + r256(2 * -(-N * K // 8192) * 4) + r256(-(-M // 8192) * 4)
            + 256 + 256 + r256(M * 4))
    o_dyt = int(C.lib().concord_sigmag_noise_workspace_bytes(M, N, K)) - rest
    o_prod = o_dyt + r256(M * N * 2)
    o_ssum = o_prod + r256(N * K * 2) + r256(2 * -(-N * K // 8192) * 4) + r256(-(-M // 8192) * 4)
    dyt = host(ws[o_dyt:o_dyt + M * N * 2].view(torch.bfloat16)).view(np.uint16).reshape(M, N)
    P = host(ws[o_prod:o_prod + N * K * 2].view(torch.bfloat16)).view(np.uint16).reshape(N, K)
    S = host(ws[o_ssum:o_ssum + 4].view(torch.float32))[0]
    eps = oracle.token_draws(313, M)
    dyf = host(dy.float())
    np.testing.assert_array_equal(dyt, oracle.f32_to_bf16_bits_array((eps[:, None] * dyf).astype(np.float32)))
    assert S.view(np.uint32) == oracle.token_sum(313, M).view(np.uint32)
    ref = oracle.bf16_bits_to_f32(dyt).astype(np.float64).T @ host(x.float()).astype(np.float64)
    assert rel_l2(oracle.bf16_bits_to_f32(P).astype(np.float64), ref) < 1e-2
    want = oracle.sigmag_combine(host(g0).view(np.uint16), P, S, M, 0.3)
    np.testing.assert_array_equal(host(g).view(np.uint16), want)
    assert int(host(salt)[0]) == 313
    # the reference forms the draw in fp32 ((eps * gy)^T x, prototype_packed_b.py:1492-1494);
    # this build rounds eps*dy and the product to bf16.  The added noise against
    # that expression in float64 (same eps, same gradient):
    g0f = oracle.bf16_bits_to_f32(host(g0).view(np.uint16)).astype(np.float64)
    n64 = (eps[:, None].astype(np.float64) * dyf.astype(np.float64)).T @ host(x.float()).astype(np.float64) \
        - float(np.float64(eps.astype(np.float64).sum())) * g0f / M
    add64 = n64 * (0.3 * np.linalg.norm(g0f) / max(np.linalg.norm(n64), 1e-12))
    added = oracle.bf16_bits_to_f32(host(g).view(np.uint16)).astype(np.float64) - g0f
    err = rel_l2(added, add64)
    print(f"Sigma_g draw against the fp32-form reference in float64: rel-L2 {err:.2e}")
    assert err < 2e-2


def test_layer_sigmag_noise_step():
    """The layer's backward with the default (Sigma_g) noise on: the update
    sees a gradient whose added part has norm sigma ||grad_W||, and two runs
    at the same salt inject the same noise."""
    import concord_amd as ca
    from concord_amd import packed_b as pb
    torch.manual_seed(14)
    x = torch.randn(512, 256, device=DEV).to(torch.bfloat16)
    gy = (torch.randn(512, 384, device=DEV) * 1e-2).to(torch.bfloat16)
    plain = pb._wgrad(gy, x).float()
    caps = []
    ca.set_sigmag_noise(True)
    ca.set_sigmag_sigma(0.25)
    try:
        for _ in range(2):
            pb._get_step_counter(DEV).fill_(600)
            layer = ca.ConcordLinearPackedB(256, 384, bias=False, device=DEV, lr=1e-3)
            cap = []
            pb._DEBUG_CAPTURE = cap
            layer(x.clone().requires_grad_(True)).backward(gy)
            pb._DEBUG_CAPTURE = None
            caps.append(cap[0].float())
    finally:
        pb._DEBUG_CAPTURE = None
        ca.set_sigmag_noise(False)
        ca.set_sigmag_sigma(0.0)
    sync()
    np.testing.assert_array_equal(host(caps[0]), host(caps[1]))
    d = (caps[0] - plain).norm().item() / plain.norm().item()
    assert abs(d - 0.25) < 1e-2, d
