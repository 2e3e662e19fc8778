"""CPU checks of the grid-barrier protocol and the work split of the WGRAD
launch that carries the v-hat finalize and the update (grid_sync, grid_exit,
upd_finalize and upd_apply in concord_amd/csrc/wgrad_update.h).

The protocol is restated with one thread per workgroup and a semaphore for
the CUs: arrivals and exits are atomic adds, a waiter gives up after its
bound and adds the poison mark, the last workgroup out re-arms the counters
and either advances the salt or raises the fault flag.  The checks: with
every workgroup resident both barriers complete and the state is re-armed
for the next launch; with fewer CUs than workgroups the waits end by the
bound, nobody writes, every workgroup still exits, the fault flag is raised
and the counters are re-armed.  The index checks: phase 2's row blocks,
bias rows and columns, and phase 3's tile elements each cover every index
exactly once for the launch shapes the host allows."""
import threading
import time

POISON = 1 << 24


class Counters:
    def __init__(self):
        self.lock = threading.Lock()
        self.bar = 0
        self.exitc = 0
        self.fault = 0
        self.salt = 5

    def add(self, name, v):
        with self.lock:
            old = getattr(self, name)
            setattr(self, name, old + v)
            return old

    def load(self, name):
        with self.lock:
            return getattr(self, name)

    def store(self, name, v):
        with self.lock:
            setattr(self, name, v)


def grid_sync(c, target, timeout_s):
    """grid_sync of wgrad_update.h: returns True when poisoned."""
    c.add("bar", 1)
    t0 = time.monotonic()
    while True:
        v = c.load("bar")
        if v >= POISON:
            return True
        if v >= target:
            return False
        if time.monotonic() - t0 > timeout_s:
            c.add("bar", POISON)
            return True
        time.sleep(0.0005)


def grid_exit(c, grid):
    e = c.add("exitc", 1)
    if e == grid - 1:
        if c.load("bar") >= POISON:
            c.store("fault", 1)
        else:
            c.store("salt", c.load("salt") + 1)
        c.store("bar", 0)
        c.store("exitc", 0)


def launch(c, grid, cus, timeout_s=0.2, work_s=0.0):
    """One launch: `grid` workgroups on `cus` CUs (a workgroup holds its CU
    until it exits).  Returns the phases each workgroup wrote in."""
    cu = threading.Semaphore(cus)
    wrote = [[] for _ in range(grid)]

    def wg(w):
        with cu:
            if work_s:
                time.sleep(work_s * (w % 3) / 2)   # uneven phase 1
            bad = grid_sync(c, grid, timeout_s)
            if not bad:
                wrote[w].append(2)
            bad2 = grid_sync(c, 2 * grid, timeout_s)
            if not bad2 and not bad:
                wrote[w].append(3)
            grid_exit(c, grid)

    ts = [threading.Thread(target=wg, args=(w,)) for w in range(grid)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=30)
        assert not t.is_alive(), "a workgroup did not exit"
    return wrote


def test_barrier_all_resident_and_rearmed():
    c = Counters()
    for k in range(3):   # consecutive launches on one workspace
        wrote = launch(c, grid=24, cus=24, work_s=0.002)
        assert all(w == [2, 3] for w in wrote)
        assert (c.bar, c.exitc, c.fault) == (0, 0, 0)
        assert c.salt == 5 + k + 1


def test_barrier_not_resident_times_out_without_writes():
    c = Counters()
    wrote = launch(c, grid=12, cus=8, timeout_s=0.05)
    # the first 8 wait for 4 workgroups that cannot start: every wait ends by
    # the bound, the late workgroups see the mark, nobody runs phase 3
    assert all(w == [] for w in wrote)
    assert c.fault == 1 and c.bar == 0 and c.exitc == 0 and c.salt == 5
    # the next launch that fits runs normally on the re-armed counters
    c.fault = 0
    wrote = launch(c, grid=8, cus=8)
    assert all(w == [2, 3] for w in wrote) and c.fault == 0 and c.salt == 6


def cdiv(a, b):
    return (a + b - 1) // b


def _phase2_cover(N, K, grid):
    """upd_finalize's split: workgroup b < rb rows b*256 + t (t < 256) and
    bias rows (t >= 256); workgroups rb.. columns (wg - rb) * 512 + t."""
    rb = cdiv(N, 256)
    rows, bias, cols = [0] * N, [0] * N, [0] * K
    for wg in range(grid):
        for t in range(512):
            if wg < rb:
                i = wg * 256 + (t & 255)
                if i < N:
                    (rows if t < 256 else bias)[i] += 1
            else:
                k = (wg - rb) * 512 + t
                if k < K:
                    cols[k] += 1
    return rows, bias, cols


def _phase3_cover(N, K):
    """upd_apply over 256 x 128 tiles of 8 waves (wi 0..3, wj 0..1), lane
    16 q + p: rows row0 + 16 x + p, columns col0 + 16 y + 4 q + e."""
    seen = {}
    for bi in range(cdiv(N, 256)):
        for bj in range(cdiv(K, 128)):
            for wi in range(4):
                for wj in range(2):
                    row0, col0 = bi * 256 + wi * 64, bj * 128 + wj * 64
                    for lane in range(64):
                        p, q = lane & 15, lane >> 4
                        for x in range(4):
                            i = row0 + 16 * x + p
                            for y in range(4):
                                j = col0 + 16 * y + 4 * q
                                if i < N and j < K:
                                    for e in range(4):
                                        assert j + e < K   # K % 8 == 0
                                        seen[(i, j + e)] = seen.get((i, j + e), 0) + 1
                    # watermark slots: rows wi*64 + 16x + p < 256, columns wj*64 + 16y + 4q + e < 128
    return seen


def test_phase_splits_cover_every_index_once():
    for N, K in ((5120, 1280), (1280, 1280), (2560, 640), (384, 256), (5120, 2816)):
        tiles = cdiv(N, 256) * cdiv(K, 128)
        grid = 256
        if tiles > grid - 16 or cdiv(N, 256) + cdiv(K, 512) > grid:
            continue   # the host does not take the combined launch
        rows, bias, cols = _phase2_cover(N, K, grid)
        assert set(rows) == {1} and set(bias) == {1} and set(cols) == {1}, (N, K)
    for N, K in ((384, 256), (520, 136)):
        seen = _phase3_cover(N, K)
        assert len(seen) == N * K and set(seen.values()) == {1}
