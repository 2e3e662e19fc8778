"""GatedRebalance with the gate on the device (concord_rebalance_group),
through the C ABI: every layer's packed words, exponents, high-watermarks
and seed must be bit-identical to the per-layer rebalance loop the gate
replaces (notebook/src/concord_winner.py:254-262), whether the gate fires or
not, eagerly and replayed from a captured HIP graph."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, host, sync

pytestmark = pytest.mark.gpu

# (out N, in K): ragged edges (rows and columns not multiples of 32 / 256),
# 1 x 1, and enough shift tiles (> 2048 in all) that the shift kernel's
# per-block ranges span several tiles and cross layer boundaries
SHAPES = [(300, 520), (1, 1), (4100, 2600), (33, 257), (1280, 5120), (3000, 3000), (65, 70),
          (2500, 4000), (256, 256)]


def _layers(seed):
    import concord_amd as ca
    torch.manual_seed(seed)
    layers = []
    for n, k in SHAPES:
        m = ca.ConcordLinearPackedB(k, n, bias=False, device=DEV)
        m.load_weights(torch.randn(n, k) / k ** 0.5)
        # spread the words over the mantissa range so shifts round
        with torch.no_grad():
            m.packed_w.copy_(torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k), dtype=torch.int64).to(torch.int32))
            m.row_exp.copy_(torch.randint(-8, 8, (n,), dtype=torch.int8))
            m.col_exp.copy_(torch.randint(-8, 8, (k,), dtype=torch.int8))
            m._reb_seed.fill_(1000 + n)
        m._ensure_buffers()
        layers.append(m)
    return layers


def _state(layers):
    return [t.clone() for m in layers for t in (m.packed_w, m.row_exp, m.col_exp, m._row_max_hwm,
                                               m._col_max_hwm, m._reb_seed)]


def _restore(layers, st):
    it = iter(st)
    for m in layers:
        for t in (m.packed_w, m.row_exp, m.col_exp, m._row_max_hwm, m._col_max_hwm, m._reb_seed):
            t.copy_(next(it))


def _assert_same(a, b):
    for x, y in zip(a, b):
        np.testing.assert_array_equal(host(x), host(y))


def _fill_watermarks(gate, rng, mode):
    """Watermarks as the update leaves them (all >= 0): 'none' below MAX_M
    everywhere, 'sparse' a few rows and columns of some layers above it,
    'dense' about one in eight above it, 'first_cols' column 0 of every layer
    above it (each layer's first shift tile fires and its last ones do not,
    so block ranges that cross into a layer start on a firing tile)."""
    nr, nc = gate.row_all.numel(), gate.col_all.numel()
    mx = gate.MAX_M
    if mx + 3000 >= 32768:
        raise AssertionError("MAX_M leaves no room above it")
    if mode == "dense":
        r = rng.integers(0, mx + 3000, nr)
        c = rng.integers(0, mx + 3000, nc)
    else:
        r = rng.integers(0, mx + 1, nr)
        c = rng.integers(0, mx + 1, nc)
        if mode == "sparse":
            r[rng.choice(nr, 7, replace=False)] = mx + 1
            c[rng.choice(nc, 5, replace=False)] = mx + 500
        elif mode == "first_cols":
            c[np.cumsum([0] + [k for _, k in SHAPES[:-1]])] = mx + 1
    gate.row_all.copy_(torch.from_numpy(r.astype(np.int32)))
    gate.col_all.copy_(torch.from_numpy(c.astype(np.int32)))
    return bool(max(r.max(), c.max()) > mx)


@pytest.mark.parametrize("mode", ["none", "sparse", "dense", "first_cols"])
def test_group_matches_per_layer_loop(mode):
    import concord_amd as ca
    layers = _layers(5)
    gate = ca.GatedRebalance(layers)
    assert gate() is False   # wires the slabs
    rng = np.random.default_rng({"none": 1, "sparse": 2, "dense": 3, "first_cols": 4}[mode])
    fire = _fill_watermarks(gate, rng, mode)
    st0 = _state(layers)
    assert gate() is None
    sync()
    got = _state(layers)
    assert gate.fires == int(fire)
    _restore(layers, st0)
    if fire:
        for m in layers:
            m.rebalance()
    sync()
    want = _state(layers)
    _assert_same(got, want)
    changed = any(not torch.equal(a, b) for a, b in zip(got, st0))
    assert changed == fire
    if fire:
        # every layer's seed advanced by one, whether or not it ticked
        seeds = [int(host(m._reb_seed)[0]) for m in layers]
        assert seeds == [1001 + n for n, _ in SHAPES]


def test_group_layer_oracle(oracle):
    """One layer of the group against the oracle's rebalance directly."""
    import concord_amd as ca
    layers = _layers(6)
    gate = ca.GatedRebalance(layers)
    gate()
    _fill_watermarks(gate, np.random.default_rng(9), "dense")
    i = 3   # 33 x 257
    m = layers[i]
    pk, re, ce = host(m.packed_w).copy(), host(m.row_exp).copy(), host(m.col_exp).copy()
    rm, cm = host(m._row_max_buf).copy(), host(m._col_max_buf).copy()
    seed = int(host(m._reb_seed)[0]) + 1
    gate()
    sync()
    oracle.rebalance(pk, re, ce, rm, cm, max_m=m.MAX_M, exp_max=m.EXP_MAX, exp_min=m.EXP_MIN, seed=seed)
    np.testing.assert_array_equal(host(m.packed_w), pk)
    np.testing.assert_array_equal(host(m.row_exp), re)
    np.testing.assert_array_equal(host(m.col_exp), ce)


def test_group_graph_replay():
    """The gate captured in a HIP graph: each replay, with new watermarks
    written eagerly in between (fire, no fire, fire, dense, first columns, no
    fire), leaves the layers as the eager per-layer loop does."""
    import concord_amd as ca
    layers = _layers(7)
    gate = ca.GatedRebalance(layers)
    gate()
    rng = np.random.default_rng(11)
    _fill_watermarks(gate, rng, "none")
    gate()   # eager call: builds the plan before capture
    sync()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    st_pre = _state(layers)
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            gate()
    torch.cuda.current_stream().wait_stream(s)
    sync()
    _assert_same(_state(layers), st_pre)   # capture ran nothing
    fires = gate.fires
    for mode in ("sparse", "none", "sparse", "dense", "first_cols", "none"):
        fire = _fill_watermarks(gate, rng, mode)
        st0 = _state(layers)
        g.replay()
        sync()
        got = _state(layers)
        fires += int(fire)
        assert gate.fires == fires
        _restore(layers, st0)
        if fire:
            for m in layers:
                m.rebalance()
        sync()
        _assert_same(got, _state(layers))
