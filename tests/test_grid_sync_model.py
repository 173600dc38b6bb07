"""CPU model of the resident quantizer's grid-wide wait
(ane_amd/csrc/quantize_fused.hip, grid_arrive_wait): the slot's tagged
64-bit counters and release words, with every workgroup's atomics as
separate steps so that arrivals of one or two launches interleave in any
order.

Checked over many random interleavings:
* one launch alone: every workgroup passes, none records an error, and the
  slot's counters end at rest (zero);
* two launches sharing the slot at once (a replayed graph overlapping
  another call): no workgroup passes its wait before every workgroup of
  its own launch has arrived unless an error bit is recorded; a launch
  whose workgroups all passed with nothing recorded has exact maxima.
A scripted overlap (a workgroup of a second launch reads its release word
just before the first launch releases) is also run on a deliberately broken
variant of the model (release words without the tag check), which the same
property must catch."""
import random

import pytest

GROUPS = 16
MIXED, TIMEOUT = 2, 1
MASK32 = (1 << 32) - 1


class Slot:
    def __init__(self, ng):
        self.top = 0
        self.err = 0
        self.gen = [0] * ng
        self.sub = [0] * ng


def workgroup(slot, partials, launch, w, G, tag, maxval, arrived, check_tag=True, timeout_polls=400):
    """Generator: one workgroup's thread 0; yields between atomics.  Returns
    (passed_on_release, bad) through StopIteration.value."""
    ng = min(G, GROUPS)
    g = w % ng
    members = (G - g + ng - 1) // ng
    gen0 = slot.gen[g]
    yield
    partials[launch][w] = maxval
    yield
    inc = (tag << 32) | 1
    old = slot.sub[g]
    slot.sub[g] = (old + inc) & ((1 << 64) - 1)
    arrived[launch].add(w)
    yield
    bad = 0

    def tags_match(v, n):
        return ((v >> 32) + tag) & MASK32 == (n * tag) & MASK32

    if old & MASK32 == members - 1:
        if not tags_match(old, members):
            bad = MIXED
        top = slot.top
        slot.top = (top + inc) & ((1 << 64) - 1)
        yield
        last = top & MASK32 == ng - 1
        if last and not tags_match(top, ng):
            bad = MIXED
        if bad:
            slot.err |= bad
            yield
        slot.sub[g] = 0
        yield
        if last:
            slot.top = 0
            yield
            rel = ((((gen0 >> 32) + 1) << 32) | tag) & ((1 << 64) - 1)
            for i in range(ng):
                slot.gen[i] = rel
                yield
            return ("releaser", bad)
    for _ in range(timeout_polls):
        v = slot.gen[g]
        if v != gen0:
            if not check_tag or v & MASK32 == tag:
                return ("released", bad)
            if not bad & MIXED:
                bad |= MIXED
                slot.err |= MIXED
        yield
    slot.err |= TIMEOUT
    return ("timeout", bad | TIMEOUT)


def run(nlaunch, G, seed, check_tag=True, stagger=0):
    rng = random.Random(seed)
    ng = min(G, GROUPS)
    slot = Slot(ng)
    partials = [[None] * G for _ in range(nlaunch)]
    arrived = [set() for _ in range(nlaunch)]
    tags = [1 + 3 * i for i in range(nlaunch)]
    maxima = [[rng.randrange(1, 1000) for _ in range(G)] for _ in range(nlaunch)]
    live = {}
    # launch l's workgroups start after `stagger * l` scheduling steps
    pending = [(l, w) for l in range(nlaunch) for w in range(G)]
    outcome = {}
    seen_at_pass = {}
    step = 0
    while pending or live:
        startable = [p for p in pending if p[0] * stagger <= step]
        if startable and (not live or rng.random() < 0.3):
            l, w = startable[rng.randrange(len(startable))]
            pending.remove((l, w))
            live[(l, w)] = workgroup(slot, partials, l, w, G, tags[l], maxima[l][w], arrived,
                                     check_tag=check_tag)
        if live:
            key = rng.choice(list(live))
            try:
                next(live[key])
            except StopIteration as e:
                outcome[key] = e.value
                l, _ = key
                seen_at_pass[key] = max(v for v in partials[l] if v is not None) \
                    if e.value[0] != "timeout" else None
                # a workgroup that passed reads its launch's partial maxima now
                seen_at_pass[key] = (len(arrived[l]) == G, seen_at_pass[key])
                del live[key]
        step += 1
    return slot, outcome, seen_at_pass, maxima


@pytest.mark.parametrize("G", [1, 3, 16, 37, 256])
def test_one_launch_passes_and_rests(G):
    for seed in range(30):
        slot, outcome, seen, maxima = run(1, G, seed)
        assert all(o[0] in ("released", "releaser") and o[1] == 0 for o in outcome.values())
        assert sum(o[0] == "releaser" for o in outcome.values()) == 1
        assert all(full for full, _ in seen.values())
        assert slot.err == 0 and slot.top == 0 and not any(slot.sub)


def _silent_early_pass(outcome, seen, slot):
    """A workgroup that passed its wait, with nothing recorded anywhere,
    before every workgroup of its launch had arrived."""
    return [k for k, (full, _) in seen.items() if not full and outcome[k][0] != "timeout" and slot.err == 0]


@pytest.mark.parametrize("G", [16, 37, 64])
@pytest.mark.parametrize("stagger", [0, 40, 400])
def test_two_launches_never_pass_silently(G, stagger):
    mixed_runs = 0
    for seed in range(60):
        slot, outcome, seen, maxima = run(2, G, seed, stagger=stagger)
        assert not _silent_early_pass(outcome, seen, slot), seed
        # a launch with nothing recorded at all has complete maxima at every pass
        if slot.err == 0:
            assert all(full for full, _ in seen.values())
        else:
            mixed_runs += 1
    if stagger == 0:
        assert mixed_runs > 0  # the interleavings do exercise the detection


def run_scripted(G, check_tag):
    """Launch 1's workgroup 0 reads its release word, then launch 0 runs to
    completion, then launch 1 runs (the overlap of a graph replay starting
    while another call's wait is ending)."""
    slot = Slot(min(G, GROUPS))
    partials = [[None] * G, [None] * G]
    arrived = [set(), set()]
    late = workgroup(slot, partials, 1, 0, G, 4, 5, arrived, check_tag=check_tag)
    next(late)  # release word read
    outcome, seen = {}, {}

    def drain(gens, launch, ids):
        live = dict(zip(ids, gens))
        while live:
            for k in list(live):
                try:
                    next(live[k])
                except StopIteration as e:
                    outcome[(launch, k)] = e.value
                    seen[(launch, k)] = (len(arrived[launch]) == G, None)
                    del live[k]

    drain([workgroup(slot, partials, 0, w, G, 1, 7, arrived, check_tag=check_tag) for w in range(G)], 0, range(G))
    # the late workgroup runs ahead of the rest of its launch for a while
    for _ in range(50):
        try:
            next(late)
        except StopIteration as e:
            outcome[(1, 0)] = e.value
            seen[(1, 0)] = (len(arrived[1]) == G, None)
            late = None
            break
    rest = [workgroup(slot, partials, 1, w, G, 4, 5, arrived, check_tag=check_tag) for w in range(1, G)]
    if late is None:
        drain(rest, 1, range(1, G))
    else:
        drain([late] + rest, 1, range(G))
    return slot, outcome, seen


@pytest.mark.parametrize("G", [16, 37, 256])
def test_foreign_release_is_recorded(G):
    """The scripted overlap: with the tag check the late workgroup records
    the foreign release and still passes on its own launch's release, every
    workgroup having arrived; without it (a planted mistake in the model)
    it passes early with nothing recorded, which the property catches."""
    slot, outcome, seen = run_scripted(G, check_tag=True)
    assert not _silent_early_pass(outcome, seen, slot)
    assert slot.err == MIXED and outcome[(1, 0)] == ("released", MIXED)
    assert all(full for full, _ in seen.values())
    slot, outcome, seen = run_scripted(G, check_tag=False)
    assert _silent_early_pass(outcome, seen, slot) == [(1, 0)]
