"""CPU check of the decode kernel's work schedule (nq_decode.hip), restated in Python.

The decode kernel cuts every row (batch, kv head, head group) into 32-key steps,
concatenates the steps of all rows and gives each wave one contiguous range of them
(a split over the launched waves weighted by the XCD each wave runs on, or an even
one when the weights would leave a wave without steps, or `chunk/32` steps per wave).  A wave that
does not cover a whole row writes an fp32 partial to slot `wave + row`; the merge
kernel combines, for each row, the partials of the waves between the first and the
last wave that covered it (both recorded by those waves).  This test restates that
integer logic on random shapes and checks the properties the kernels rely on:
every step is covered exactly once, no two partials share a slot, every slot is
below `waves + rows` (the workspace size), and the merge's wave range is exactly
the set of waves that touched the row.  The GPU tests check the kernels' outputs.
"""

import random

import pytest

STEP = 32
WAVES = 4                 # waves per workgroup
EVEN_W, ODD_W = 25, 22    # persistent split: weight of a wave on an even / odd XCD


def _split_weight(w):
    """Total weight of waves [0, w) (workgroup i runs on XCD i mod 8)."""
    gw = WAVES * 8
    rounds, k = divmod(w, gw)
    g, r = divmod(k, WAVES)
    return (rounds * WAVES * 4 * (EVEN_W + ODD_W) + (((g + 1) // 2) * EVEN_W + (g // 2) * ODD_W) * WAVES
            + r * (ODD_W if g & 1 else EVEN_W))


def _steps(length, max_len):
    n = min(length, max_len)
    return (n + STEP - 1) // STEP if n > 0 else 0


def _check(B, Hkv, G, lens, max_len, chunk, resident=1024):
    NG = (G + 15) // 16
    rows_per_batch = Hkv * NG
    R = B * rows_per_batch
    span = (chunk + STEP - 1) // STEP if chunk > 0 else 0
    if span == 0:
        launched, nwaves = 1024, resident
    else:
        upper = R * ((max_len + STEP - 1) // STEP)
        launched = ((upper + span - 1) // span + 3) // 4 * 4
        nwaves = launched
    nb = [_steps(x, max_len) for x in lens]
    N = sum(nb) * rows_per_batch
    if N == 0:
        return
    used = (N + span - 1) // span if span else min(nwaves, N)
    if span:
        begin = lambda w: min(N, w * span)  # noqa: E731
    elif N * ODD_W >= _split_weight(used):  # weighted, while every wave still gets a step
        begin = lambda w: _split_weight(w) * N // _split_weight(used)  # noqa: E731
    else:
        begin = lambda w: w * N // used  # noqa: E731

    covered = [0] * N
    slots, whole_rows, touched, first_w, last_w = {}, set(), {}, {}, {}
    for w in range(min(nwaves, used)):
        q0, q1 = begin(w), begin(w + 1)
        if q0 >= q1:
            continue
        run, b = 0, None
        for bb in range(B):
            v = nb[bb] * rows_per_batch
            if v > 0 and run <= q0 < run + v:
                b, before = bb, run
                break
            run += v
        assert b is not None
        n = nb[b]
        j, ls = divmod(q0 - before, n)
        q = q0
        while True:
            nseg = min(n - ls, q1 - q)
            assert nseg > 0
            r = b * rows_per_batch + j
            start = sum(nb[:b]) * rows_per_batch + j * n + ls
            for s in range(start, start + nseg):
                covered[s] += 1
            touched.setdefault(r, set()).add(w)
            if ls == 0:
                first_w[r] = w
            if ls + nseg == n:
                last_w[r] = w
            if ls == 0 and nseg == n:
                whole_rows.add(r)
            else:
                slot = w + r
                assert slot < launched + R
                assert slot not in slots, f"slot {slot} used by {slots[slot]} and {(w, r)}"
                slots[slot] = (w, r)
            q += nseg
            if q >= q1:
                break
            ls, j = 0, j + 1
            if j == rows_per_batch:
                j = 0
                b += 1
                while nb[b] == 0 and b + 1 < B:
                    b += 1
                n = nb[b]
                assert n > 0
    assert all(c == 1 for c in covered)
    if not span:  # every launched wave of the split holds at least one step
        assert all(begin(w + 1) > begin(w) for w in range(used))
    for r in range(R):
        if nb[r // rows_per_batch] == 0:
            assert r not in touched
            continue
        wf, wl = first_w[r], last_w[r]
        assert set(range(wf, wl + 1)) == touched[r]
        assert (wf == wl) == (r in whole_rows)
        for w in range(wf, wl + 1):
            if wf != wl:
                assert slots[w + r] == (w, r)


def test_split_weights():
    """The weights the closed form sums: waves of even workgroups EVEN_W, of odd ones ODD_W."""
    acc = 0
    for w in range(3 * WAVES * 8 + 5):
        assert _split_weight(w) == acc
        acc += ODD_W if (w // WAVES) % 2 else EVEN_W


def test_bench_and_test_shapes():
    rng = random.Random(5)
    _check(64, 4, 16, [rng.randint(1024, 32768) for _ in range(64)], 32768, 0)
    _check(64, 4, 16, [rng.randint(1024, 32768) for _ in range(64)], 32768, 1024)
    for chunk in (32, 64, 0):
        _check(4, 1, 16, [1, 100, 300, 64], 300, chunk)
    _check(3, 8, 1, [2100, 1025, 33], 2100, 0)
    _check(3, 1, 32, [2100, 1025, 33], 2100, 0)
    for chunk in (32, 256, 1024, 8192):
        _check(2, 2, 8, [5000, 3333], 5000, chunk)


@pytest.mark.parametrize("seed", range(4))
def test_random_shapes(seed):
    rng = random.Random(100 + seed)
    for _ in range(60):
        B = rng.randint(1, 150)
        Hkv = rng.choice([1, 2, 4, 8])
        G = rng.choice([1, 2, 4, 8, 16, 32, 48])
        max_len = rng.randint(1, 3000)
        lens = [rng.choice([0, -3, rng.randint(1, max_len + 50)]) if rng.random() < 0.2
                else rng.randint(1, max_len) for _ in range(B)]
        _check(B, Hkv, G, lens, max_len, rng.choice([0, 0, 32, 64, 100, 1024, 4096]),
               rng.choice([1024, 512, 8, 1]))
