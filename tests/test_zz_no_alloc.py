"""concord_rebalance_noalloc: the rebalance entry point whose scratch is a
static device array instead of a caller workspace.  Its results must equal
concord_rebalance's bit for bit (packed words, exponents, high-watermarks,
seed), over two calls in a row on one device, the second on a smaller layer
(the static scratch keeps the first call's contents), with and without the
tick-down path; sizes beyond the static scratch are refused before any
launch."""
import numpy as np
import pytest
import torch

from gpu_util import DEV, dev, host, rand_state, sync

pytestmark = pytest.mark.gpu

MAX_DIM = 131072


def _noalloc():
    from concord_amd import _lib as C
    return C.lib().concord_rebalance_noalloc


def _case(rng, N, K):
    packed, re, ce = rand_state(rng, N, K, exp=(-8, 7), col=(-3, 3))
    rm = rng.integers(0, 30000, N).astype(np.int32)
    cm = rng.integers(0, 30000, K).astype(np.int32)
    return packed, re, ce, rm, cm


def _run(entry, case, tickdown):
    from concord_amd import _lib as C
    from concord_amd import packed_b as pb
    packed, re, ce, rm, cm = case
    N, K = packed.shape
    t = [dev(packed), dev(re), dev(ce), dev(rm), dev(cm), torch.zeros(N, dtype=torch.int32, device=DEV),
         torch.zeros(K, dtype=torch.int32, device=DEV), torch.full((1,), 41, dtype=torch.int32, device=DEV)]
    pk, red, ced, rmd, cmd, rh, ch, seed = t
    st = C.stream_of(torch.device(DEV))
    args = [C.ptr(pk), K, C.ptr(red), C.ptr(ced), C.ptr(rmd), C.ptr(cmd), C.ptr(rh), C.ptr(ch), C.ptr(seed), N, K,
            24000, 7, -8, int(tickdown), 1]
    if entry == "workspace":
        ws = pb._workspace(torch.device(DEV), N, K)
        rc = C.lib().concord_rebalance(*args, C.ptr(ws), ws.numel(), st)
    else:
        rc = _noalloc()(*args, st)
    assert rc == 0, C.lib().concord_last_error()
    sync()
    return [host(x) for x in (pk, red, ced, rh, ch, seed)]


@pytest.mark.parametrize("tickdown", [False, True])
def test_noalloc_rebalance_matches_workspace_entry(tickdown):
    rng = np.random.default_rng(91 + tickdown)
    first = _case(rng, 1536, 2304)
    second = _case(rng, 300, 520)     # smaller: the scratch still holds the first call's values
    for case in (first, second):
        want = _run("workspace", case, tickdown)
        got = _run("noalloc", case, tickdown)
        for w, g in zip(want, got):
            np.testing.assert_array_equal(g, w)
        assert (want[0] != case[0]).any() and (want[1] != case[1]).any()   # some rows ticked


def test_noalloc_rebalance_refuses_oversized_layers():
    from concord_amd import _lib as C
    f = _noalloc()
    dummy = torch.zeros(16, dtype=torch.int32, device=DEV)
    p = C.ptr(dummy)
    st = C.stream_of(torch.device(DEV))
    rc = f(p, MAX_DIM + 1, p, p, p, p, p, p, p, 4, MAX_DIM + 1, 24000, 7, -8, 0, 1, st)
    assert rc == C.EINVAL
    assert b"static scratch" in C.lib().concord_last_error()
    rc = f(p, 16, p, p, p, p, p, p, p, MAX_DIM + 1, 16, 24000, 7, -8, 0, 1, st)
    assert rc == C.EINVAL
    sync()
    assert int(host(dummy).sum()) == 0
