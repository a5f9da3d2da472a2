"""Host logic of the continuous-batching decode driver (gi_batch_*) and of
the batched AppendToken it uses (gi_kvmgr_append_batch), without a device.

The model: a running set is a dense list of sequences; a step is one
AppendToken per running sequence in row order (PagedKVManager.AppendToken,
pkg/engine/paged_kv.go:107-132, copy-on-write form for forked sequences);
removing a sequence moves the last row into its place.  After every step the
driver's rows, lengths and block-table mirror must equal the model and the
manager's own tables, and the batched append must match the oracle's
restated PagedKVManager doing the same appends one by one."""
import random

import numpy as np
import pytest


def _check_against_manager(drv, mgr, model_rows):
    ids, lens = drv.Rows()
    assert list(ids) == model_rows
    for r, sid in enumerate(model_rows):
        t = mgr.Tables[sid]
        assert int(lens[r]) == t.NumTokens
        assert list(drv.RowTable(r)) == list(t.BlockIDs)


def test_append_batch_matches_oracle_lifo(gi, oracle):
    """Without forks the batched append is AppendToken in order: the same
    block ids and slots as the reference allocator's LIFO pops."""
    mgr = gi.PagedKVManager(2, 64, 40, 4)
    ref = oracle.PagedKVManager(2, 64, 40, 4)
    a = [mgr.AllocateSequence() for _ in range(3)]
    b = [ref.AllocateSequence() for _ in range(3)]
    for step in range(12):
        ids, slots, cf = mgr.AppendBatch(a)
        want = [ref.AppendToken(s) for s in b]
        assert [(int(x), int(y)) for x, y in zip(ids, slots)] == want, step
        assert not (cf >= 0).any()
    assert mgr.FreeBlocks == ref.FreeBlocks


def test_append_batch_all_or_nothing(gi):
    mgr = gi.PagedKVManager(1, 64, 5, 4)
    s = [mgr.AllocateSequence() for _ in range(3)]
    mgr.AppendBatch(s)                      # 3 blocks taken, 2 left
    for _ in range(3):
        mgr.AppendBatch(s)                  # fill the blocks (4 tokens each)
    before = (mgr.FreeBlocks, [mgr.Tables[x].BlockIDs for x in s], [mgr.Tables[x].NumTokens for x in s])
    with pytest.raises(gi.GIError) as e:    # the next token needs 3 new blocks
        mgr.AppendBatch(s)
    assert e.value.code == -4
    after = (mgr.FreeBlocks, [mgr.Tables[x].BlockIDs for x in s], [mgr.Tables[x].NumTokens for x in s])
    assert before == after
    for bad, code in (([s[0], s[0]], -3), ([s[0], 999], -6)):
        with pytest.raises(gi.GIError) as e:
            mgr.AppendBatch(bad)
        assert e.value.code == code
        assert [mgr.Tables[x].NumTokens for x in s] == [4, 4, 4]
    mgr.FreeSequence(s[2])                  # 1 block comes back: 3 free now
    ids, slots, cf = mgr.AppendBatch(s[:2])
    assert list(slots) == [0, 0]


def test_driver_random_schedule(gi):
    """Joins, leaves, forks (copy-on-write) and steps at random."""
    rng = random.Random(11)
    P, N = 4, 200
    mgr = gi.PagedKVManager(1, 64, N, P)
    drv = gi.BatchDecoder(mgr, None, 12, N)
    rows = []
    pending_copy = {}
    exhausted = [0]
    for it in range(400):
        op = rng.random()
        if op < 0.15 and len(rows) < 12:
            n = rng.randrange(0, 30)
            if (n + P - 1) // P > len(mgr.FreeBlocks):
                continue
            sid = mgr.AllocateSequence()
            if n:
                mgr.AppendTokens(sid, n)
            assert drv.Add(sid) == len(rows)
            rows.append(sid)
        elif op < 0.22 and rows:
            sid = rows[rng.randrange(len(rows))]
            r = rows.index(sid)
            drv.Remove(sid)
            rows[r] = rows[-1]
            rows.pop()
            mgr.FreeSequence(sid)
        elif op < 0.3 and rows and len(rows) < 12:
            src = rows[rng.randrange(len(rows))]
            n = mgr.Tables[src].NumTokens
            f = mgr.ForkSequence(src, rng.randrange(0, n + 1))
            drv.Add(f)
            rows.append(f)
        else:
            free_before = len(mgr.FreeBlocks)
            shared = {s: (mgr.Tables[s].BlockIDs[-1] if mgr.Tables[s].BlockIDs else -1) for s in rows}
            try:
                n = drv.Step()
            except gi.GIError as e:
                # refused whole: nothing changed; preempt one sequence
                assert e.code == -4
                _check_against_manager(drv, mgr, rows)
                sid = rows[-1]
                drv.Remove(sid)
                rows.pop()
                mgr.FreeSequence(sid)
                exhausted[0] += 1
                continue
            assert n == len(rows)
            # a copied block replaced a shared last block in place
            for s in rows:
                t = mgr.Tables[s]
                if t.NumTokens % P != 1 and shared[s] >= 0 and t.BlockIDs[-1] != shared[s]:
                    pending_copy[s] = (shared[s], t.BlockIDs[-1])
            assert len(mgr.FreeBlocks) <= free_before
        _check_against_manager(drv, mgr, rows)
    assert pending_copy, "the schedule should have exercised copy-on-write steps"
    assert exhausted[0] > 0, "the schedule should have run the pool dry at least once"
    drv.close()


def test_driver_errors(gi):
    mgr = gi.PagedKVManager(1, 64, 8, 4)
    drv = gi.BatchDecoder(mgr, None, 2, 2)
    a, b, c = (mgr.AllocateSequence() for _ in range(3))
    drv.Add(a)
    with pytest.raises(gi.GIError):
        drv.Add(a)                             # already running
    with pytest.raises(gi.GIError) as e:
        drv.Add(999)                           # unknown sequence
    assert e.value.code == -6
    drv.Add(b)
    with pytest.raises(gi.GIError):
        drv.Add(c)                             # batch full
    with pytest.raises(gi.GIError) as e:
        drv.Remove(c)                          # not running
    assert e.value.code == -6
    for _ in range(8):
        drv.Step()                             # 8 tokens = 2 blocks each
    with pytest.raises(gi.GIError) as e:       # a 9th token outgrows max_blocks
        drv.Step()
    assert e.value.code == -3
    ids, lens = drv.Rows()
    assert list(lens) == [8, 8]
    with pytest.raises(gi.GIError):
        drv.DecodeLayer(0, 8, None, None, None, None, 1.0)  # no device pool
    drv.Remove(a)
    assert list(drv.Rows()[0]) == [b]


def test_append_batch_shared_block_exact_capacity(gi):
    """Two forks and their source share a partial last block (3 references):
    a step over all three takes 2 copies, not 3, so it fits a pool with
    exactly 2 free blocks."""
    mgr = gi.PagedKVManager(1, 64, 3, 4)
    a = mgr.AllocateSequence()
    mgr.AppendTokens(a, 2)                   # 1 block, half full; 2 free
    b, c = mgr.ForkSequence(a, 2), mgr.ForkSequence(a, 2)
    shared = mgr.Tables[a].BlockIDs[0]
    assert mgr.BlockRefs(shared) == 3 and len(mgr.FreeBlocks) == 2
    ids, slots, cf = mgr.AppendBatch([a, b, c])
    assert sorted(int(x) for x in cf if x >= 0) == [shared, shared]
    assert list(slots) == [2, 2, 2]
    assert len(mgr.FreeBlocks) == 0
    assert len({int(x) for x in ids}) == 3     # three distinct blocks now
