"""The prefix-cache restatement (oracle/prefix_cache.py) against cases worked out by hand from
src/worker.rs:115-174: the strict-prefix rule, live continuation, restore only when a snapshot
beats the live hit, the snapshot_at window, LRU eviction with empty slots first and the first
minimum on a tie, and the dropping of snapshots whose attention entries a request overwrites."""
from prefix_cache import PrefixCache, shared_prefix


def test_shared_prefix_is_strict():
    assert shared_prefix([1, 2], [1, 2, 3]) == 2
    assert shared_prefix([1, 2, 3], [1, 2, 3]) == 0  # equal: at least one token must be fed
    assert shared_prefix([1, 2, 3, 4], [1, 2, 3]) == 0
    assert shared_prefix([1, 3], [1, 2, 3]) == 0
    assert shared_prefix([], [7]) == 0


def test_first_request_resets_then_live_continues():
    c = PrefixCache()
    d = c.begin([1, 2, 3])
    assert (d["action"], d["cached"], d["feed_from"]) == ("reset", 0, 0)
    c.decoded([7, 8])  # e.g. an accepted draft fed both
    d = c.begin([1, 2, 3, 7, 8, 9])
    assert (d["action"], d["cached"], d["feed_from"]) == ("live", 5, 5)
    c.decoded([])
    # the same prompt again is not a strict extension of the live keys: start over
    d = c.begin([1, 2, 3, 7, 8, 9])
    assert (d["action"], d["cached"]) == ("reset", 0)


def test_snapshot_window_and_restore():
    c = PrefixCache()
    s = [5, 6, 7, 8]
    d = c.begin(s + [1, 1], snapshot_at=4)
    assert (d["snapshot_slot"], d["feed_from"]) == (0, 4)
    c.decoded([9])
    assert c.state() == (7, [4, -1, -1, -1], [1, 0, 0, 0])
    # another continuation of s: the live keys diverge at position 4, slot 0 covers 4 tokens
    d = c.begin(s + [2, 2, 2], snapshot_at=4)  # snapshot_at not past the reused part: none
    assert (d["action"], d["slot"], d["cached"], d["snapshot_slot"]) == ("restore", 0, 4, None)
    assert c.state()[2][0] == 2  # restoring refreshes the slot's clock
    c.decoded([])
    # snapshot_at must stay short of the prompt
    d = c.begin(s + [2, 2, 2, 3], snapshot_at=8)
    assert (d["action"], d["cached"], d["snapshot_slot"]) == ("live", 7, None)


def test_restore_only_when_it_beats_the_live_hit():
    c = PrefixCache()
    p = list(range(10, 20))
    c.begin(p, snapshot_at=6)  # slot 0 holds p[:6]
    c.decoded([])
    # live (10 keys) is a strict prefix and longer than the snapshot: continue live
    d = c.begin(p + [1])
    assert (d["action"], d["cached"]) == ("live", 10)
    c.decoded([])
    # a prompt sharing exactly the snapshot's keys with the live ones beyond: snapshot wins
    d = c.begin(p[:6] + [0, 0])
    assert (d["action"], d["slot"], d["cached"]) == ("restore", 0, 6)


def test_lru_eviction_over_nested_turns():
    c = PrefixCache()
    seq = []
    for turn in range(5):
        seq = seq + [100 + 10 * turn + k for k in range(4)]
        d = c.begin(seq, snapshot_at=len(seq) - 1)
        assert d["snapshot_slot"] == (turn if turn < 4 else 0)  # empty slots first, then the oldest
        c.decoded([])
    assert c.state() == (20, [19, 7, 11, 15], [5, 2, 3, 4])
    # branch off the second turn's snapshot (slot 1, 7 keys): the longer snapshots are not
    # prefixes of the new prompt and their attention entries get overwritten, so they go
    d = c.begin(seq[:7] + [1, 2, 3], snapshot_at=8)
    assert (d["action"], d["slot"], d["cached"]) == ("restore", 1, 7)
    # slots 0, 2, 3 were emptied; the snapshot at 8 goes to the first empty one
    assert d["snapshot_slot"] == 0
    assert c.state() == (10, [8, 7, -1, -1], [6, 6, 0, 0])
    c.decoded([4])
    # a tie on last use between slots 0 and 1 after filling the rest: the first one goes
    d = c.begin(seq[:7] + [1, 2, 3, 4, 5, 6], snapshot_at=12)
    assert d["snapshot_slot"] == 2
    c.decoded([])
    d = c.begin(seq[:7] + [1, 2, 3, 4, 5, 6, 7, 8], snapshot_at=14)
    assert d["snapshot_slot"] == 3
    c.decoded([])
    d = c.begin(seq[:7] + [1, 2, 3, 4, 5, 6, 7, 8, 9, 9], snapshot_at=16)
    assert d["snapshot_slot"] == 0
    assert c.state()[1:] == ([16, 7, 12, 14], [9, 6, 7, 8])


def test_unrelated_prompt_drops_overwritten_snapshots():
    c = PrefixCache()
    a = [1, 2, 3, 4, 5]
    c.begin(a + [6], snapshot_at=5)
    c.decoded([7])
    d = c.begin([1, 2, 9, 9])  # shares 2 keys with the snapshot, then writes other entries
    assert (d["action"], d["cached"]) == ("reset", 0)
    assert c.state()[1] == [-1, -1, -1, -1]
    c.decoded([])
    d = c.begin(a + [8])
    assert (d["action"], d["cached"]) == ("reset", 0)


def test_snapshot_equal_to_prompt_survives():
    c = PrefixCache()
    s = [3, 1, 4, 1]
    c.begin(s + [5], snapshot_at=4)
    c.decoded([])
    d = c.begin([3, 1, 4, 1])  # resets (nothing is a strict prefix) but writes the same keys
    assert d["action"] == "reset"
    assert c.state()[1][0] == 4
    c.decoded([2])
    d = c.begin(s + [9, 9])
    assert (d["action"], d["slot"], d["cached"]) == ("restore", 0, 4)


def test_error_clears_everything():
    c = PrefixCache()
    c.begin([1, 2, 3, 4], snapshot_at=2)
    c.error()
    assert c.state() == (0, [-1, -1, -1, -1], [0, 0, 0, 0])
