"""Host side of the device block-table mirror (CPU only): the native step_metadata against its
Python restatement on random step sequences (appends, releases, re-use of states, hand edits of
a block list, row take-over), the descriptor it writes checked against each request's actual
block list, and the row assignment (free on state deletion, least-recently-used take-over)."""
import gc
import random

import numpy as np
import pytest
import torch

from src.cache.paged_kv import LayerBlockPool, PagedKVCacheState
from src.model.graph_decode import _BlockTableMirror, _step_metadata_py

try:
    from src.cache import _paged_host as native
except ImportError:  # pragma: no cover - the build makes it
    native = None

LAYOUT_B = 6
W = 20


def layout(B, stride):
    o_cur, o_sel, o_mrow, o_first, o_npages = 0, B, 2 * B, 3 * B, 4 * B
    o_prev, o_app, o_upd = 5 * B, 6 * B, 7 * B
    return (o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, stride), o_upd + B * stride


def reconstruct(desc, lay, B, dev_rows):
    """Apply a descriptor to a model of the device mirror; return each request's block list."""
    o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, stride = lay
    lists = []
    for b in range(B):
        row, f, n = desc[o_mrow + b], desc[o_first + b], desc[o_npages + b]
        upd = list(desc[o_upd + b * stride:o_upd + b * stride + n - f])
        full = list(dev_rows[row][:f]) + upd
        dev_rows[row][f:n] = upd
        lists.append(full)
    return lists


@pytest.mark.skipif(native is None, reason="native host module not built")
def test_native_step_metadata_matches_python_and_reconstructs_lists():
    rng = random.Random(5)
    R = 8
    mir_py = (np.full((R, W), -1, np.int32), np.zeros(R, np.int32))
    mir_nat = (np.full((R, W), -1, np.int32), np.zeros(R, np.int32))
    dev_rows = np.full((R, W), -7, np.int64)  # what the device mirror holds (applied descriptors)
    lists = {i: [] for i in range(10)}
    for step in range(300):
        B = rng.randint(1, LAYOUT_B)
        reqs = rng.sample(sorted(lists), B)
        for r in reqs:
            op = rng.random()
            if op < 0.6:
                lists[r] = lists[r] + [rng.randrange(1000) for _ in range(rng.randint(0, 3))]
            elif op < 0.7:
                lists[r] = []  # released
            elif op < 0.8 and lists[r]:
                lists[r] = list(lists[r])
                lists[r][rng.randrange(len(lists[r]))] = rng.randrange(1000)  # edited by hand
            lists[r] = lists[r][:W]
        states = [PagedKVCacheState(pool=None, block_ids=list(lists[r])) for r in reqs]
        rows = [r % R for r in reqs]  # distinct within a step (requests 0..9 over 8 rows: r, r+8 collide)
        if len(set(rows)) != len(rows):
            continue
        if rng.random() < 0.05:
            for t in (mir_py, mir_nat):
                t[1][rows[0]] = 0  # the row was taken over: resend
        prev = [rng.randint(0, 300) for _ in reqs]
        app = [rng.randint(0, 16) for _ in reqs]
        cur = [rng.randint(-2, 20) for _ in reqs]
        sel = [rng.randint(0, 15) for _ in reqs]
        lay, words = layout(B, W)
        d_py = np.zeros(words, np.int32)
        d_nat = np.zeros(words, np.int32)
        got_py = _step_metadata_py(states, rows, prev, app, cur, sel, mir_py[0], mir_py[1], d_py, lay)
        got_nat = native.step_metadata(states, rows, prev, app, cur, sel, mir_nat[0], mir_nat[1], d_nat, lay)
        assert tuple(got_py) == tuple(got_nat)
        assert np.array_equal(d_py, d_nat), step
        assert np.array_equal(mir_py[0], mir_nat[0]) and np.array_equal(mir_py[1], mir_nat[1])
        # the descriptor rebuilds every request's list on the device model of the mirror
        assert reconstruct(d_nat, lay, B, dev_rows) == [lists[r] for r in reqs], step
        o_cur, o_sel, _, _, _, o_prev, o_app, _, _ = lay
        assert list(d_nat[o_cur:o_cur + B]) == cur and list(d_nat[o_sel:o_sel + B]) == sel
        assert list(d_nat[o_prev:o_prev + B]) == prev and list(d_nat[o_app:o_app + B]) == app


@pytest.mark.parametrize("impl", ["py", "native"])
def test_step_metadata_errors(impl):
    if impl == "native" and native is None:
        pytest.skip("native host module not built")
    fn = _step_metadata_py if impl == "py" else native.step_metadata
    lay, words = layout(1, 4)
    shadow, slen = np.full((2, 4), -1, np.int32), np.zeros(2, np.int32)
    st = [PagedKVCacheState(pool=None, block_ids=[1, 2, 3, 4, 5])]
    with pytest.raises(ValueError, match="mirror width"):
        fn(st, [0], [0], [0], [0], [0], shadow, slen, np.zeros(words, np.int32), lay)
    st = [PagedKVCacheState(pool=None, block_ids=[1])]
    with pytest.raises(ValueError, match="mirror row"):
        fn(st, [2], [0], [0], [0], [0], shadow, slen, np.zeros(words, np.int32), lay)


def test_mirror_rows_follow_states():
    pool = LayerBlockPool(16, 4, 2.0)
    mir = _BlockTableMirror(3, 8, torch.device("cpu"))  # the row bookkeeping does not touch the device copy
    a, b, c, d = (PagedKVCacheState(pool=pool) for _ in range(4))
    assert mir.rows_for([a, b]) == [0, 1]
    mir.shadow_len[:] = [5, 6, 0]
    assert mir.rows_for([b, a]) == [1, 0] and list(mir.shadow_len[:2]) == [5, 6]  # kept
    assert mir.rows_for([c]) == [2]
    # no free row: d takes over the least recently used row not used in this step
    rd = mir.rows_for([d, c])
    assert rd[1] == 2 and rd[0] in (0, 1) and mir.shadow_len[rd[0]] == 0
    taken = rd[0]
    survivor = b if taken == 0 else a
    assert mir.rows_for([survivor]) == [1 - taken]
    # the request whose row was taken gets a row again, resent whole
    loser = a if taken == 0 else b
    r = mir.rows_for([loser])[0]
    assert mir.shadow_len[r] == 0
    # a state that is garbage collected frees its row
    e = PagedKVCacheState(pool=pool)
    re_ = mir.rows_for([e])[0]
    assert not mir._free
    del e
    gc.collect()
    assert mir._free == [re_] and re_ not in mir._row_of.values()
    assert mir.rows_for([PagedKVCacheState(pool=pool) for _ in range(4)]) is None  # more states than rows
