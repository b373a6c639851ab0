"""Model check of the scan's decoupled-lookback descriptor protocol (CPU).

A randomized scheduler interleaves, one memory word at a time, what the
tiles of one scan do in kernelforge.jl_amd/csrc/kf_scan.hip:
  * tiles are numbered by workgroup id and start in dispatch order: tile t
    queues on XCD t mod X, each XCD starts its queue in increasing order and
    holds at most a few tiles at once (a tile leaves when it is done);
  * a started tile "loads" its aggregate, publishes PARTIAL (W tagged
    words, written one by one in random order), looks back, publishes PREFIX;
  * a lookback poll reads the descriptors of a window of predecessors, each
    word separately (so a reader can observe a half-written descriptor), and
    applies the kernel's acceptance rules: a descriptor is valid only when
    every word carries the current epoch and the same state; the walk stops
    at the newest PREFIX if every tile after it is valid, moves one window
    back if the whole window is valid PARTIALs, and otherwise polls again.
The operator is string concatenation (non-commutative and non-idempotent), so
any wrong order, duplicated or dropped tile shows up in the final prefixes.
Memory starts with descriptors of earlier calls (older epochs), which must
be ignored. This checks the protocol the kernel implements, on schedules a
GPU run cannot force.
"""
import random

import pytest

INVALID, PARTIAL, PREFIX = 0, 1, 2


class Memory:
    def __init__(self, ntiles, W, stale_epoch, rng):
        # stale words from an earlier call: random states and values, old epoch
        self.words = {}
        for t in range(ntiles):
            for w in range(W):
                st = rng.choice([INVALID, PARTIAL, PREFIX])
                self.words[(t, w)] = ((stale_epoch << 2) | st, f"<stale{t}.{w}>")


def split_words(value, W):
    """A value spread over W words (the kernel splits T into 32-bit words)."""
    k = max(1, -(-len(value) // W))
    parts = [value[i * k:(i + 1) * k] for i in range(W)]
    return parts


def classify(words, epoch):
    """The kernel's acceptance rule: (state, value) of one descriptor."""
    tags = {wd[0] for wd in words}
    ok = len(tags) == 1 and (next(iter(tags)) >> 2) == epoch
    return ((next(iter(tags)) & 3) if ok else INVALID), "".join(wd[1] for wd in words)


def classify_word0_only(words, epoch):
    """A broken rule that trusts word 0's tag alone (accepts torn reads)."""
    tag = words[0][0]
    return ((tag & 3) if (tag >> 2) == epoch else INVALID), "".join(wd[1] for wd in words)


def tile_program(t, agg, mem, epoch, W, window, rng, result, accept=classify):
    """Generator: one memory word access per step (a scheduler interleaves)."""
    tag = lambda st: (epoch << 2) | st

    def publish(state, value):
        order = list(range(W))
        rng.shuffle(order)
        parts = split_words(value, W)
        for w in order:
            mem.words[(t, w)] = (tag(state), parts[w])
            yield

    if t == 0:
        yield from publish(PREFIX, agg)
        result[t] = ""
        return
    yield from publish(PARTIAL, agg)
    run = ""
    newest = t - 1
    while True:
        lanes = []
        for lane_t in range(newest - window + 1, newest + 1):
            if lane_t < 0:
                lanes.append((PREFIX, ""))
                continue
            words = []
            for w in range(W):
                words.append(mem.words[(lane_t, w)])
                yield
            lanes.append(accept(words, epoch))
        states = [s for s, _ in lanes]
        prefix_lanes = [i for i, s in enumerate(states) if s == PREFIX]
        if prefix_lanes:
            m = prefix_lanes[-1]
            if all(s != INVALID for s in states[m:]):
                run = "".join(v for _, v in lanes[m:]) + run
                break
        elif all(s != INVALID for s in states):
            run = "".join(v for _, v in lanes) + run
            newest -= window
            continue
        yield  # sleep, then poll again
    result[t] = run
    yield from publish(PREFIX, run + agg)


class Stuck(Exception):
    """No tile can make progress: the dispatch order deadlocked."""


def run_schedule(seed, W, accept=classify, reverse_xcd_order=False, max_steps=400_000):
    rng = random.Random(seed * 7 + W)
    ntiles = rng.randint(1, 40)
    window = rng.choice([1, 2, 8, 64])
    epoch = rng.randint(1, 1000)
    mem = Memory(ntiles, W, epoch - rng.randint(1, 3), rng)
    aggs = [f"[{t}]" for t in range(ntiles)]
    result = {}
    nxcd = rng.choice([1, 2, 8])
    slots = rng.randint(1, 3)   # tiles one XCD holds at once
    queues = [[t for t in range(ntiles) if t % nxcd == x] for x in range(nxcd)]
    if reverse_xcd_order:
        queues = [q[::-1] for q in queues]
    running = [set() for _ in range(nxcd)]
    progs = {}
    steps = 0
    while any(queues) or progs:
        steps += 1
        if steps > max_steps:
            raise Stuck(f"seed {seed}: {len(progs)} tiles waiting, {sum(map(len, queues))} not started")
        free = [x for x in range(nxcd) if queues[x] and len(running[x]) < slots]
        if free and (not progs or rng.random() < 0.3):
            x = rng.choice(free)
            t = queues[x].pop(0)
            running[x].add(t)
            progs[t] = tile_program(t, aggs[t], mem, epoch, W, window, rng, result, accept)
            continue
        t = rng.choice(list(progs))
        try:
            next(progs[t])
        except StopIteration:
            del progs[t]
            running[t % nxcd].discard(t)
    return ntiles, epoch, aggs, result, mem


@pytest.mark.parametrize("seed", range(40))
@pytest.mark.parametrize("W", [1, 2])
def test_lookback_protocol_random_schedules(seed, W):
    ntiles, epoch, aggs, result, mem = run_schedule(seed, W)
    for t in range(ntiles):
        assert result[t] == "".join(aggs[:t]), (t, result[t])
    # every descriptor ends as this epoch's PREFIX holding the inclusive prefix
    for t in range(ntiles):
        words = [mem.words[(t, w)] for w in range(W)]
        assert all(wd[0] == (epoch << 2) | PREFIX for wd in words)
        assert "".join(wd[1] for wd in words) == "".join(aggs[:t + 1])


def test_model_detects_a_broken_acceptance_rule():
    # negative control: trusting one word of a two-word descriptor must
    # produce a wrong prefix on some schedule, or the model proves nothing
    wrong = 0
    for seed in range(200):
        ntiles, _, aggs, result, _ = run_schedule(seed, 2, accept=classify_word0_only)
        wrong += any(result[t] != "".join(aggs[:t]) for t in range(ntiles))
    assert wrong > 0


def test_model_detects_out_of_order_dispatch():
    # negative control for the progress argument: if an XCD started its
    # workgroups in decreasing id order, a full XCD of tiles waiting on a
    # lower tile it has not started would never drain
    stuck = 0
    for seed in range(30):
        try:
            run_schedule(seed, 1, reverse_xcd_order=True, max_steps=20_000)
        except Stuck:
            stuck += 1
    assert stuck > 0


def test_torn_descriptor_is_rejected():
    # word 0 already PREFIX, word 1 still PARTIAL: INVALID, not a mixed value
    epoch = 5
    torn = [((epoch << 2) | PREFIX, "[0][1"), ((epoch << 2) | PARTIAL, "]")]
    assert classify(torn, epoch)[0] == INVALID
    stale = [(((epoch - 1) << 2) | PREFIX, "x"), (((epoch - 1) << 2) | PREFIX, "y")]
    assert classify(stale, epoch)[0] == INVALID
    fresh = [((epoch << 2) | PARTIAL, "[3"), ((epoch << 2) | PARTIAL, "]")]
    assert classify(fresh, epoch) == (PARTIAL, "[3]")
