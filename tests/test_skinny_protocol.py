"""Model check of the one-launch skinny kernels' slot protocols (CPU).

``k_skinny`` (csrc/skinny.hip) and ``k_skinny_one`` (csrc/skinny2.hip) hand
partial results between the blocks of one launch through a slot of arrival
words, and a call only works if the slot is all-zero when it starts. Each
block is modelled here as a sequence of atomic operations on the slot words
(the fetch-adds, loads and stores of the kernels, in program order; a
bounded wait is a run of loads that gives up after ``spin`` polls), and a
scheduler interleaves the blocks at random. For every schedule, including
those where a wait expires because the blocks it waits for have not run
yet, the slot must be all-zero once every block has finished, and a wait
that succeeded must only have succeeded on this call's own arrivals.

The protocol the kernels used before (the last finisher clears the adapter
word; a late adapter then increments it again) is kept as a negative
control: the checker must find the schedules that leave its slot dirty.
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
    arrivals, [1] done, [2 + t] split arrivals of tile t."""

    done_target = adapters + tiles

    def done_count():
        old = slot.fetch_add(1)
        if old + 1 == done_target:
            slot.w[0] = 0
            yield
            slot.w[1] = 0
        yield

    def adapter():
        slot.fetch_add(0)
        yield
        if fixed:
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
        ok = snapshot == adapters
        polls = 0
        while not ok and polls < spin:
            ok = slot.w[0] == adapters
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


def skinny_one_blocks(slot: Slot, adapters: int, weights: int, spin: int, log: list,
                      fixed: bool = True):
    """Generators for the blocks of one k_skinny_one launch. Words: [0]
    adapter arrivals, [1] h published, [2] done."""

    done_target = weights + 1

    def done_count():
        old = slot.fetch_add(2)
        if old + 1 == done_target:
            slot.w[0] = 0
            yield
            slot.w[1] = 0
            yield
            slot.w[2] = 0
        yield

    def adapter():
        old = slot.fetch_add(0)
        last = old + 1 == adapters
        if last:
            slot.w[0] = 0
        yield
        if not last:
            return
        slot.w[1] = 1  # h published
        yield
        if fixed:
            yield from done_count()

    def weight():
        ok = False
        polls = 0
        while not ok and polls < spin:
            ok = slot.w[1] != 0
            polls += 1
            yield
        log.append(("weight", ok))
        if fixed:
            yield from done_count()
        else:
            old = slot.fetch_add(2)
            if old + 1 == weights:
                slot.w[2] = 0
                slot.w[1] = 0
            yield

    return [adapter() for _ in range(adapters)] + [weight() for _ in range(weights)]


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


def _calls(kind: str, fixed: bool, seed: int, n_calls: int = 6):
    """Runs n_calls launches on one slot back to back (a stream's order);
    returns (slot clean after every call, every successful wait legitimate)."""

    rng = random.Random(seed)
    slot = Slot(2 + 3 if kind == "skinny" else 3)
    clean = True
    legit = True
    for _ in range(n_calls):
        if any(slot.w):
            clean = False
        log: list = []
        spin = rng.choice([1, 2, 3, 50])
        late = rng.random() < 0.5
        start = list(slot.w)
        if kind == "skinny":
            adapters, tiles, splits = rng.choice([(1, 1, 2), (2, 2, 2), (3, 3, 1), (2, 3, 3)])
            gens = skinny_blocks(slot, adapters, tiles, splits, spin, log, fixed)
        else:
            adapters, weights = rng.choice([(1, 1), (2, 3), (3, 2), (4, 4)])
            gens = skinny_one_blocks(slot, adapters, weights, spin, log, fixed)
        run(gens, rng, late)
        # a wait that succeeds on a dirty slot may have counted stale arrivals
        # (k_skinny) or seen the previous call's h flag (k_skinny_one)
        if any(start):
            legit = legit and not any(entry[-1] for entry in log)
    if any(slot.w):
        clean = False
    return clean, legit


@pytest.mark.parametrize("kind", ["skinny", "skinny_one"])
def test_slot_returns_to_zero_under_every_schedule(kind):
    for seed in range(3000):
        clean, legit = _calls(kind, fixed=True, seed=seed)
        assert clean and legit, (kind, seed)


@pytest.mark.parametrize("kind", ["skinny", "skinny_one"])
def test_checker_catches_the_former_protocol(kind):
    """Negative control: the protocol without the done count leaves the slot
    dirty after an expired wait, in some schedules."""

    dirty = sum(not _calls(kind, fixed=False, seed=seed)[0] for seed in range(3000))
    assert dirty > 0


def test_slot_is_clean_when_no_wait_expires():
    """With unbounded waits (spin large, blocks interleaved fairly) both
    protocols leave the slot clean; the fix changes only the expired case."""

    for seed in range(500):
        rng = random.Random(seed)
        for fixed in (True, False):
            slot = Slot(5)
            log: list = []
            run(skinny_blocks(slot, 2, 2, 2, 10_000, log, fixed), rng, adapters_late=False)
            assert not any(slot.w) and all(ok for _, _, ok in log)
            slot = Slot(3)
            log = []
            run(skinny_one_blocks(slot, 3, 2, 10_000, log, fixed), rng, adapters_late=False)
            assert not any(slot.w) and all(ok for _, ok in log)
