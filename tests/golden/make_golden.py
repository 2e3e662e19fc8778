"""Write golden input/output vectors from the reference's own kernels.

Runs ONLY in the build container, where the reference checkout is mounted at
/root/reference (override with CONCORD_REFERENCE).  The reference's Triton
kernels are executed by Triton's CPU interpreter (TRITON_INTERPRET=1) on CPU
tensors; the resulting vectors are committed as small .npz fixtures next to
this script and read by tests/test_oracle_golden.py.  Nothing here runs on the
GPU box and nothing from the reference is copied: only inputs and outputs.

Functions covered (the ones no closed form or invariant pins bitwise):
  concord/packed_b.py           _apply_packed_adamw_kernel (422-703),
                                _apply_packed_sgd_kernel (173-312),
                                _rebalance_packed_decide_kernel (959-1095),
                                ConcordLinearPackedB.load_weights (1570-1603),
                                ConcordLinearPackedB.load_weights_finetune (1816-1856)
  notebook/src/prototype_packed_b.py  _apply_packed_adamw_kernel (454-778)

Usage:  python tests/golden/make_golden.py
"""
import os
import sys

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402

REF = os.environ.get("CONCORD_REFERENCE", "/root/reference")
OUT = os.path.dirname(os.path.abspath(__file__))


def _bf16_bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def _state(gen, N, K, sf_lo=-3000, sf_hi=3000, exp_lo=-3, exp_hi=3, col_lo=-1, col_hi=1):
    sf = torch.randint(sf_lo, sf_hi, (N, K), generator=gen, dtype=torch.int32)
    # a few elements near the int16 limits
    m = torch.rand((N, K), generator=gen) < 0.02
    sf[m] = torch.randint(-32768, 32767, (int(m.sum()),), generator=gen, dtype=torch.int32)
    ss = torch.randint(-128, 128, (N, K), generator=gen, dtype=torch.int32)
    vs = torch.randint(-128, 128, (N, K), generator=gen, dtype=torch.int32)
    packed = (((sf & 0xFFFF) << 16) | ((ss & 0xFF) << 8) | (vs & 0xFF)).to(torch.int32)
    re = torch.randint(exp_lo, exp_hi + 1, (N,), generator=gen, dtype=torch.int32).to(torch.int8)
    ce = torch.randint(col_lo, col_hi + 1, (K,), generator=gen, dtype=torch.int32).to(torch.int8)
    return packed, re, ce


def _grad(gen, N, K, lo=-5, hi=-1):
    mag = torch.pow(10.0, torch.empty(N, 1).uniform_(lo, hi, generator=gen))
    g = torch.randn((N, K), generator=gen) * mag
    g[torch.rand((N, K), generator=gen) < 0.05] = 0.0
    return g.to(torch.bfloat16)


def _vhat_inputs(gen, N, K):
    v_row = torch.rand(N, generator=gen) * 1e-3 + 1e-6
    v_col = torch.rand(K, generator=gen) * 1e-3 + 1e-6
    sum_v_inv = torch.tensor([1.0 / float(v_row.sum())], dtype=torch.float32)
    return v_row.float(), v_col.float(), sum_v_inv


def _pow4_vhat(gen, N, K):
    """v_row, v_col, sum_v_inv all powers of four -> v_hat a power of four, so
    (v_hat + 0)^0.5 is exact under any exp2/log2 implementation."""
    v_row = torch.pow(4.0, torch.randint(-12, -4, (N,), generator=gen).float())
    v_col = torch.pow(4.0, torch.randint(-12, -4, (K,), generator=gen).float())
    sum_v_inv = torch.tensor([4.0 ** 3], dtype=torch.float32)
    return v_row, v_col, sum_v_inv


def run_adamw(ppb, case, gen, N, K, lr, salt, flags, **kw):
    packed, re, ce = _state(gen, N, K, **kw.pop("state", {}))
    grad = _grad(gen, N, K, **kw.pop("grad", {}))
    pow4 = kw.pop("pow4", False)
    v_row, v_col, sum_v_inv = (_pow4_vhat if pow4 else _vhat_inputs)(gen, N, K)
    coh_pre = None
    if flags.get("cohpre"):
        coh_pre = torch.rand((N, K), generator=gen).float()
    wbuf = torch.zeros((N, K), dtype=torch.bfloat16)
    rmax = torch.zeros(N, dtype=torch.int32)
    cmax = torch.zeros(K, dtype=torch.int32)
    inputs = dict(packed=packed.numpy().copy(), grad=_bf16_bits(grad),
                  row_exp=re.numpy().copy(), col_exp=ce.numpy().copy(),
                  v_row=v_row.numpy().copy(), v_col=v_col.numpy().copy(),
                  sum_v_inv=sum_v_inv.numpy().copy(),
                  coh_pre=(coh_pre.numpy().copy() if coh_pre is not None
                           else np.zeros(0, np.float32)))
    ppb._STEP_COUNTERS.clear()
    ppb._STEP_COUNTERS[str(packed.device)] = torch.tensor([salt - 1], dtype=torch.int32)
    ppb.set_fixed_coh(flags.get("fixed_coh", True))
    ppb.set_gate_gain(kw.get("gate_gain", 1.0))
    ppb.set_ratio_coh(flags.get("ratio_coh", False))
    ppb.set_ratio_coh_floors(kw.get("chase_floor", 0.9), kw.get("leak_floor", 0.999))
    extra = {}
    if kw.get("proto"):
        ppb.set_consolidate(packed.device, bool(kw.get("consolidate", 1)))
        ppb._V_BC_BUFS.clear()
        ppb._v_bc_buf(packed.device).fill_(kw.get("v_bc", 1.0))
    args = dict(lr=lr, mantissa_bias=15, alpha=kw.get("alpha", 0.1), beta1=kw.get("beta1", 0.0),
                weight_decay=kw.get("weight_decay", 0.0), eps=kw.get("eps", 1e-10),
                step_cap=kw.get("step_cap", 10.0), v_scale=kw.get("v_scale", 0.0),
                precond_p=0.5, gf_consol=kw.get("gf_consol", 0.0),
                drift_cancel_C=kw.get("drift_cancel_C", 0.018036072144288578),
                alpha_v_fast=kw.get("alpha_v_fast", 0.001), wd_sv=kw.get("wd_sv", 0.0),
                wd_sf=kw.get("wd_sf", 0.0), mass_preserve=flags.get("mass_preserve", True),
                apply_chase=flags.get("apply_chase", True),
                track_rebalance=flags.get("track", True),
                v_row=v_row, v_col=v_col, sum_v_inv=sum_v_inv,
                gf_trust_delta_sq=kw.get("gf_trust_delta_sq", 1.0), coh_pre=coh_pre)
    args.update(extra)
    pk = packed.clone()
    ppb.apply_packed_adamw(pk, grad, wbuf, re, ce, rmax, cmax, **args)
    outputs = dict(packed_out=pk.numpy().copy(), weight_out=_bf16_bits(wbuf),
                   row_max=rmax.numpy().copy(), col_max=cmax.numpy().copy(),
                   coh_pre_out=(coh_pre.numpy().copy() if coh_pre is not None
                                else np.zeros(0, np.float32)))
    scal = dict(lr=lr, salt=salt, alpha=args["alpha"], beta1=args["beta1"],
                weight_decay=args["weight_decay"], eps=args["eps"], step_cap=args["step_cap"],
                v_scale=args["v_scale"], gf_consol=args["gf_consol"],
                drift_cancel_C=args["drift_cancel_C"], alpha_v_fast=args["alpha_v_fast"],
                wd_sv=args["wd_sv"], wd_sf=args["wd_sf"],
                gf_trust_delta_sq=args["gf_trust_delta_sq"], gate_gain=kw.get("gate_gain", 1.0),
                chase_floor=kw.get("chase_floor", 0.9), leak_floor=kw.get("leak_floor", 0.999),
                consolidate=kw.get("consolidate", 1), v_bc=kw.get("v_bc", 1.0),
                proto=int(bool(kw.get("proto"))),
                mass_preserve=int(args["mass_preserve"]), apply_chase=int(args["apply_chase"]),
                track=int(args["track_rebalance"]), fixed_coh=int(flags.get("fixed_coh", True)),
                ratio_coh=int(flags.get("ratio_coh", False)),
                cohpre=int(coh_pre is not None))
    np.savez_compressed(os.path.join(OUT, f"adamw_{case}.npz"),
                        **inputs, **outputs, **{f"s_{k}": np.array(v) for k, v in scal.items()})
    print(f"adamw_{case}: N={N} K={K} changed={(pk != packed).float().mean():.3f}")


def run_sgd(ppb, case, gen, N, K, lr, salt, mass_preserve):
    packed, re, ce = _state(gen, N, K)
    grad = _grad(gen, N, K)
    wbuf = torch.zeros((N, K), dtype=torch.bfloat16)
    rmax = torch.zeros(N, dtype=torch.int32)
    cmax = torch.zeros(K, dtype=torch.int32)
    ppb._STEP_COUNTERS.clear()
    ppb._STEP_COUNTERS[str(packed.device)] = torch.tensor([salt - 1], dtype=torch.int32)
    pk = packed.clone()
    ppb.apply_packed_sgd(pk, grad, wbuf, re, ce, rmax, cmax, lr=lr, mantissa_bias=15,
                         alpha=0.1, beta1=0.05, alpha_v_fast=0.001,
                         mass_preserve=mass_preserve, track_rebalance=True)
    np.savez_compressed(os.path.join(OUT, f"sgd_{case}.npz"), packed=packed.numpy(),
                        grad=_bf16_bits(grad), row_exp=re.numpy(), col_exp=ce.numpy(),
                        packed_out=pk.numpy(), weight_out=_bf16_bits(wbuf),
                        row_max=rmax.numpy(), col_max=cmax.numpy(), s_lr=np.array(lr),
                        s_salt=np.array(salt), s_mass_preserve=np.array(int(mass_preserve)),
                        s_alpha=np.array(0.1), s_beta1=np.array(0.05),
                        s_alpha_v_fast=np.array(0.001))
    print(f"sgd_{case}: changed={(pk != packed).float().mean():.3f}")


def run_rebalance(ppb, case, gen, N, K, seed, allow_tickdown, big_rows, big_cols, small=False):
    if small:
        sf = torch.randint(-20, 20, (N, K), generator=gen, dtype=torch.int32)
        ss = torch.randint(-14, 15, (N, K), generator=gen, dtype=torch.int32)
        vs = torch.randint(-14, 15, (N, K), generator=gen, dtype=torch.int32)
    else:
        sf = torch.randint(-3000, 3000, (N, K), generator=gen, dtype=torch.int32)
        ss = torch.randint(-60, 60, (N, K), generator=gen, dtype=torch.int32)
        vs = torch.randint(-60, 60, (N, K), generator=gen, dtype=torch.int32)
        # overflow only at (big_rows x big_cols) and along the diagonal of
        # big_rows: those rows and columns fire, the rest do not
        for r in big_rows:
            for c in list(big_cols) + [r % K]:
                ss[r, c] = 120
                vs[r, c] = 110 if (r + c) % 2 else -128 + 0 * c
                if vs[r, c] < 0:
                    ss[r, c] = -128
                    vs[r, c] = -120
    packed = (((sf & 0xFFFF) << 16) | ((ss & 0xFF) << 8) | (vs & 0xFF)).to(torch.int32)
    re = torch.randint(-2, 8, (N,), generator=gen, dtype=torch.int32).to(torch.int8)
    ce = torch.randint(-2, 8, (K,), generator=gen, dtype=torch.int32).to(torch.int8)
    if small:
        re.fill_(3)
        ce.fill_(2)
    m = ss * 128 + sf + vs * 128
    rmax = m.abs().amax(1).to(torch.int32)
    cmax = m.abs().amax(0).to(torch.int32)
    seed_buf = torch.tensor([seed], dtype=torch.int32)
    pk, re2, ce2 = packed.clone(), re.clone(), ce.clone()
    ppb.rebalance_packed(pk, re2, ce2, rmax, cmax, MAX_M=24000, EXP_MAX=7, EXP_MIN=-8,
                         seed_buf=seed_buf, allow_tickdown=allow_tickdown)
    np.savez_compressed(os.path.join(OUT, f"rebalance_{case}.npz"), packed=packed.numpy(),
                        row_exp=re.numpy(), col_exp=ce.numpy(), row_max=rmax.numpy(),
                        col_max=cmax.numpy(), packed_out=pk.numpy(), row_exp_out=re2.numpy(),
                        col_exp_out=ce2.numpy(), s_seed=np.array(seed),
                        s_allow_tickdown=np.array(int(allow_tickdown)))
    print(f"rebalance_{case}: rows_up={(re2 > re).sum()} cols_up={(ce2 > ce).sum()} "
          f"rows_dn={(re2 < re).sum()} changed={(pk != packed).float().mean():.3f}")


def run_load(ppb, gen):
    torch.manual_seed(0)
    N, K = 40, 72
    W = torch.randn((N, K), generator=gen) * torch.pow(10.0, torch.empty(N, 1).uniform_(-4, 1.5, generator=gen))
    W[3] = 0.0
    W[5, :] = 0.25          # exact power of two max
    W[6, 0] = -1.0
    W[7] *= 1e4             # clamps at EXP_MAX
    layer = ppb.ConcordLinearPackedB(K, N, bias=False, device="cpu")
    layer.load_weights(W)
    p1, r1, c1 = layer.packed_w.numpy().copy(), layer.row_exp.numpy().copy(), layer.col_exp.numpy().copy()
    layer.load_weights_finetune(W)
    p2, r2, c2 = layer.packed_w.numpy().copy(), layer.row_exp.numpy().copy(), layer.col_exp.numpy().copy()
    np.savez_compressed(os.path.join(OUT, "load_weights.npz"), W=W.numpy(), packed=p1, row_exp=r1,
                        col_exp=c1, packed_ft=p2, row_exp_ft=r2, col_exp_ft=c2)
    print("load_weights: ok")


def main():
    sys.path.insert(0, REF)
    import concord.packed_b as ppb  # noqa: E402
    gen = torch.Generator().manual_seed(1234)
    N, K = 48, 80
    run_adamw(ppb, "bare", gen, N, K, 5e-4, 17, dict(cohpre=True))
    run_adamw(ppb, "bare_pow4", gen, N, K, 5e-4, 18, dict(cohpre=True),
              pow4=True, eps=0.0)
    run_adamw(ppb, "winner", gen, N, K, 5e-4, 19, dict(ratio_coh=True), gf_consol=50.0,
              chase_floor=0.7, leak_floor=0.95)
    run_adamw(ppb, "winner_pow4", gen, N, K, 3e-3, 20, dict(ratio_coh=True), gf_consol=50.0,
              chase_floor=0.3, leak_floor=0.5, pow4=True, eps=0.0)
    run_adamw(ppb, "wd_legacy", gen, N, K, 1e-2, 21,
              dict(fixed_coh=False, cohpre=True, mass_preserve=False),
              weight_decay=0.01, wd_sv=0.3, wd_sf=0.2, beta1=0.05, v_scale=1.0,
              gate_gain=0.8, eps=1.0)
    run_adamw(ppb, "nochase_notrust", gen, N, K, 1e-3, -5,
              dict(apply_chase=False, track=False), gf_trust_delta_sq=0.0, eps=1.0, v_scale=1.0)
    run_adamw(ppb, "big", gen, 100, 200, 2e-4, 123456, dict(cohpre=True),
              state=dict(exp_lo=-8, exp_hi=7, col_lo=-3, col_hi=3))
    run_sgd(ppb, "mp", gen, N, K, 0.05, 33, True)
    run_sgd(ppb, "nomp", gen, N, K, 0.01, 34, False)
    run_rebalance(ppb, "up", gen, 64, 96, 5, False, big_rows=[3, 17, 40], big_cols=[7, 70])
    run_rebalance(ppb, "up_td", gen, 64, 96, 6, True, big_rows=[1, 2], big_cols=[95])
    run_rebalance(ppb, "tickdown", gen, 64, 64, 7, True, [], [], small=True)
    run_load(ppb, gen)

    sys.path.insert(0, os.path.join(REF, "notebook", "src"))
    import prototype_packed_b as proto  # noqa: E402
    run_adamw(proto, "proto_winner", gen, N, K, 5e-4, 40, dict(ratio_coh=True), gf_consol=50.0,
              chase_floor=0.6, leak_floor=0.9, proto=True, consolidate=1, v_bc=1.25, beta1=0.1)
    run_adamw(proto, "proto_accum", gen, N, K, 5e-4, 41, dict(ratio_coh=True), gf_consol=50.0,
              chase_floor=0.6, leak_floor=0.9, proto=True, consolidate=0, v_bc=1.0, beta1=0.1)
    run_adamw(proto, "proto_pow4", gen, N, K, 2e-3, 42, dict(ratio_coh=True), gf_consol=20.0,
              chase_floor=0.5, leak_floor=0.5, proto=True, consolidate=1, v_bc=4.0, beta1=0.1,
              pow4=True, eps=0.0)


if __name__ == "__main__":
    main()
