"""Restatement of the generation worker's prefix-cache decisions (src/worker.rs:115-174).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the shipped library.

For each request the worker either continues the state the caches hold ("live"), restores the
snapshot whose keys are the longest strict prefix of the prompt, or resets; it may then snapshot
part-way through the prompt into the least recently used slot.  Rust's `max_by_key` keeps the
LAST maximum and `min_by_key` the FIRST minimum; both tie rules are kept.

One rule is added to the reference's: a snapshot holds only the recurrent state, while the
attention caches are shared by every sequence, so once a request writes positions at or past
`cached` with keys that differ from a snapshot's, that snapshot is dropped.  The reference keeps
it and would later restore it over attention entries of another sequence.

Parity: pinned by hand-derived cases in tests/test_prefix_cache.py (strict-prefix rule, both
tie rules, LRU order, the snapshot_at window, the dropping rule), and on the GPU against the
C++ worker's own bookkeeping and token streams.
"""
from __future__ import annotations

from typing import List, Optional, Sequence

SNAPSHOTS = 4


def shared_prefix(cached: Sequence[int], prompt: Sequence[int]) -> int:
    """src/worker.rs:115-120: len(cached) if cached is a strict prefix of prompt, else 0."""
    if len(cached) < len(prompt) and list(prompt[:len(cached)]) == list(cached):
        return len(cached)
    return 0


class PrefixCache:
    def __init__(self, slots: int = SNAPSHOTS):
        self.live: List[int] = []
        self.snaps: List[Optional[tuple]] = [None] * slots  # (keys, last used)
        self.clock = 0

    def begin(self, prompt: Sequence[int], snapshot_at: Optional[int] = None) -> dict:
        """Decisions of Worker::run before decoding (src/worker.rs:139-176).  Returns
        {"action": "restore"|"reset"|"live", "slot", "cached", "snapshot_slot", "feed_from"}."""
        prompt = list(prompt)
        n = len(prompt)
        self.clock += 1
        live_hit = shared_prefix(self.live, prompt)
        best = None
        for i, s in enumerate(self.snaps):
            if s is None:
                continue
            k = shared_prefix(s[0], prompt)
            if best is None or k >= best[1]:  # max_by_key: the last maximum
                best = (i, k)
        out = {"action": "live", "slot": None, "snapshot_slot": None}
        if best is not None and best[1] > live_hit:
            slot = best[0]
            keys = self.snaps[slot][0]
            self.snaps[slot] = (keys, self.clock)
            self.live = list(keys)
            out.update(action="restore", slot=slot)
        elif live_hit == 0:
            self.live = []
            out["action"] = "reset"
        cached = len(self.live)
        out["cached"] = cached
        # the rule added to the reference's (module docstring)
        for i, s in enumerate(self.snaps):
            if s is not None and len(s[0]) > cached and (len(s[0]) > n or prompt[:len(s[0])] != list(s[0])):
                self.snaps[i] = None
        if snapshot_at is not None and len(self.live) < snapshot_at < n:
            used = [0 if s is None else s[1] for s in self.snaps]
            slot = used.index(min(used))  # min_by_key: the first minimum
            self.live = prompt[:snapshot_at]
            self.snaps[slot] = (list(self.live), self.clock)
            out["snapshot_slot"] = slot
        out["feed_from"] = len(self.live)
        self.live = prompt
        return out

    def decoded(self, fed: Sequence[int]) -> None:
        """Tokens fed during decoding (every emitted token but a final one that ended the loop)."""
        self.live = self.live + list(fed)

    def error(self) -> None:
        """src/worker.rs:94-101: a failed request leaves nothing cached."""
        self.live = []
        self.snaps = [None] * len(self.snaps)

    def state(self):
        return len(self.live), [(-1 if s is None else len(s[0])) for s in self.snaps], \
            [(0 if s is None else s[1]) for s in self.snaps]
