"""Model check of the skinny kernels' cross-block hand-offs (CPU).

``k_skinny`` (csrc/skinny.hip) hands partial results between the blocks of
one launch through a slot of arrival words, and a call only works if the
slot is all-zero when it starts. Each block is modelled here as a sequence
of atomic operations on the slot words (the fetch-adds, loads and stores of
the kernel, in program order; a bounded wait is a run of loads that gives
up after ``spin`` polls), and a scheduler interleaves the blocks at random.
For every schedule, including those where a wait expires because the
blocks it waits for have not run yet, the slot must be all-zero once every
block has finished, and a wait that succeeded must only have succeeded on
this call's own arrivals. The last adapter block to arrive counts the
adapter word once more after it has summed every adapter partial, and the
finishers wait for that count. The protocol the kernel used before (the last
finisher clears the adapter word; a late adapter then increments it again)
is kept as a negative control: the checker must find the schedules that
leave its slot dirty.

``k_skinny_one`` (csrc/skinny2.hip) needs no clean-up: every partial travels
as one word holding its value and the launch's tag, a hash of the dispatch
(the queue's dispatch id and the packet address) and the host's call
count, and a weight block takes a word only when the word carries its own
launch's tag. Modelled with the tag as the pair (dispatch, host count),
back-to-back launches and graph replays (the same host count, a new
dispatch) must never read a word of an earlier launch. A tag made of the
host's call count alone is the negative control: a replayed launch then
takes the words its previous replay left.
"""

from __future__ import annotations

import random

import pytest


class Slot:
    def __init__(self, words: int):
        self.w = [0] * words

    def fetch_add(self, i: int) -> int:
        old = self.w[i]
        self.w[i] = old + 1
        return old


def skinny_blocks(slot: Slot, adapters: int, tiles: int, splits: int, spin: int, log: list,
                  fixed: bool = True):
    """Generators for the blocks of one k_skinny launch. Words: [0] adapter
    arrivals (and, with ``fixed``, one more count from the last adapter
    once it has summed the partials), [1] done, [2 + t] split arrivals of
    tile t."""

    done_target = adapters + tiles
    h_target = adapters + 1 if fixed else adapters

    def done_count():
        old = slot.fetch_add(1)
        if old + 1 == done_target:
            slot.w[0] = 0
            yield
            slot.w[1] = 0
        yield

    def adapter():
        old = slot.fetch_add(0)
        yield
        if fixed:
            if old + 1 == adapters:
                # the last arrival sums the partials, then counts once more
                yield
                slot.fetch_add(0)
                yield
            yield from done_count()

    def weight(t: int):
        snapshot = slot.w[0]  # read with the arrival, in one round trip
        old = slot.fetch_add(2 + t)
        last = old + 1 == splits
        if last:
            slot.w[2 + t] = 0
        yield
        if not last:
            return
        ok = snapshot == h_target
        polls = 0
        while not ok and polls < spin:
            ok = slot.w[0] == h_target
            polls += 1
            yield
        log.append(("finisher", t, ok))
        if fixed:
            yield from done_count()
        else:
            old = slot.fetch_add(1)
            if old + 1 == tiles:
                slot.w[1] = 0
                slot.w[0] = 0
            yield

    gens = [adapter() for _ in range(adapters)]
    gens += [weight(t) for t in range(tiles) for _ in range(splits)]
    return gens


def skinny_one_blocks(words: dict, tag, launch: int, adapters: int, weights: int, spin: int,
                      log: list):
    """Generators for the blocks of one k_skinny_one launch (number
    ``launch``). ``words`` maps a partial's index (one per adapter block
    here) to (tag, launch that wrote it); each adapter block stores its word
    once, each weight block polls every word until all carry ``tag`` (at most
    ``spin`` polls) and logs whether the words it accepted were this
    launch's."""

    def adapter(i: int):
        yield
        words[i] = (tag, launch)
        yield

    def weight():
        seen = {}
        polls = 0
        while True:
            for i in range(adapters):
                if i not in seen and words.get(i, (0, None))[0] == tag:
                    seen[i] = words[i][1]
            polls += 1
            if len(seen) == adapters or polls >= spin:
                break
            yield
        ok = len(seen) == adapters
        log.append(("weight", ok, ok and all(w == launch for w in seen.values())))
        yield

    return [adapter(i) for i in range(adapters)] + [weight() for _ in range(weights)]


def run(gens, rng: random.Random, adapters_late: bool) -> None:
    """Interleave the blocks. With ``adapters_late`` the weight blocks get
    most turns first, so waits expire."""

    live = list(gens)
    while live:
        if adapters_late and rng.random() < 0.85:
            idx = rng.randrange(len(live) // 2, len(live)) if len(live) > 1 else 0
        else:
            idx = rng.randrange(len(live))
        try:
            next(live[idx])
        except StopIteration:
            live.pop(idx)


def _calls(fixed: bool, seed: int, n_calls: int = 6):
    """Runs n_calls k_skinny launches on one slot back to back (a stream's
    order); returns (slot clean after every call, every successful wait
    legitimate)."""

    rng = random.Random(seed)
    slot = Slot(2 + 3)
    clean = True
    legit = True
    for _ in range(n_calls):
        if any(slot.w):
            clean = False
        log: list = []
        spin = rng.choice([1, 2, 3, 50])
        late = rng.random() < 0.5
        start = list(slot.w)
        adapters, tiles, splits = rng.choice([(1, 1, 2), (2, 2, 2), (3, 3, 1), (2, 3, 3)])
        run(skinny_blocks(slot, adapters, tiles, splits, spin, log, fixed), rng, late)
        # a wait that succeeds on a dirty slot may have counted stale arrivals
        if any(start):
            legit = legit and not any(entry[-1] for entry in log)
    if any(slot.w):
        clean = False
    return clean, legit


def _one_calls(dispatch_tags: bool, seed: int, n_calls: int = 8):
    """Launches of k_skinny_one on one slot, some of them replays of the
    previous launch (same host call count); returns whether every weight
    block that accepted words accepted only its own launch's."""

    rng = random.Random(seed)
    words: dict = {}
    host = 0
    dispatch = 0
    legit = True
    for i in range(n_calls):
        if i == 0 or rng.random() < 0.5:
            host += 1  # a new call; otherwise a graph replay of the last one
        dispatch += 1
        tag = (dispatch, host) if dispatch_tags else host
        log: list = []
        adapters, weights = rng.choice([(1, 1), (2, 3), (3, 2), (4, 4)])
        spin = rng.choice([1, 2, 3, 50])
        run(skinny_one_blocks(words, tag, i, adapters, weights, spin, log), rng,
            adapters_late=rng.random() < 0.5)
        legit = legit and all(own for _, ok, own in log if ok)
    return legit


def test_skinny_slot_returns_to_zero_under_every_schedule():
    for seed in range(3000):
        clean, legit = _calls(fixed=True, seed=seed)
        assert clean and legit, seed


def test_checker_catches_the_former_skinny_protocol():
    """Negative control: the protocol without the done count leaves the slot
    dirty after an expired wait, in some schedules."""

    dirty = sum(not _calls(fixed=False, seed=seed)[0] for seed in range(3000))
    assert dirty > 0


def test_skinny_one_takes_only_its_own_launchs_words():
    """Dispatch-derived tags: no schedule, replay or expired wait lets a
    launch read a word that an earlier launch left in the slot."""

    for seed in range(3000):
        assert _one_calls(dispatch_tags=True, seed=seed), seed


def test_checker_catches_host_only_tags_on_replays():
    """Negative control: with the host's call count as the tag, a graph
    replay takes the words of its previous replay in some schedules."""

    stale = sum(not _one_calls(dispatch_tags=False, seed=seed) for seed in range(3000))
    assert stale > 0


def test_slot_is_clean_when_no_wait_expires():
    """With unbounded waits (spin large, blocks interleaved fairly) both
    k_skinny protocols leave the slot clean; the fix changes only the
    expired case. k_skinny_one's waits all succeed on their own words."""

    for seed in range(500):
        rng = random.Random(seed)
        for fixed in (True, False):
            slot = Slot(5)
            log: list = []
            run(skinny_blocks(slot, 2, 2, 2, 10_000, log, fixed), rng, adapters_late=False)
            assert not any(slot.w) and all(ok for _, _, ok in log)
        words: dict = {}
        for call in range(3):
            log = []
            run(skinny_one_blocks(words, (call, 1), call, 3, 2, 10_000, log), rng,
                adapters_late=False)
            assert all(ok and own for _, ok, own in log)
