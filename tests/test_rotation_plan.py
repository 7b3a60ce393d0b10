"""Rotation planner and compact-plaintext bound against the reference's headers.

Expected values come from tests/golden/rotation_steps.json, recorded by
tests/golden/make_rotation_fixture.py from the reference's
native/fideslib_stage0/include/rotation_steps.hpp and plaintext_rns.hpp.
"""
import json
import os
import random

import pytest

from fhemamba_amd.plaintext import compact_plaintext_fits
from fhemamba_amd.rotation import (RotationBatchStats, canonical_rotation, naf_steps,
                                   rotate_prefix_batch, rotation_steps)

HERE = os.path.dirname(os.path.abspath(__file__))
with open(os.path.join(HERE, "golden", "rotation_steps.json")) as fh:
    FIX = json.load(fh)


@pytest.mark.parametrize("value,expected", FIX["naf"])
def test_naf_steps_match_reference(value, expected):
    if expected is None:
        with pytest.raises(OverflowError):
            naf_steps(value)
    else:
        assert naf_steps(value) == expected


@pytest.mark.parametrize("offset,slots,naf,expected", FIX["rotation_steps"])
def test_rotation_steps_match_reference(offset, slots, naf, expected):
    assert rotation_steps(offset, slots, bool(naf)) == expected


@pytest.mark.parametrize("slots,scale,q0,values,expected", FIX["compact_fits"])
def test_compact_fits_matches_reference(slots, scale, q0, values, expected):
    assert compact_plaintext_fits(values, slots, scale, q0) == bool(expected)


def test_naf_properties():
    # sum reproduces the value, digits non-adjacent, magnitudes ascending
    for v in list(range(-2000, 2001)) + [2**30 - 1, -(2**30) + 7]:
        steps = naf_steps(v)
        assert sum(steps) == v
        mags = [abs(s) for s in steps]
        assert mags == sorted(mags)
        for a, b in zip(mags, mags[1:]):
            assert b >= 4 * a  # no two adjacent nonzero digits
        assert all(m & (m - 1) == 0 for m in mags)


def test_canonical_rotation_range():
    for slots in (2, 4, 64, 1024):
        for off in range(-3 * slots, 3 * slots):
            c = canonical_rotation(off, slots)
            assert -slots // 2 <= c <= slots // 2
            assert (c - off) % slots == 0
    with pytest.raises(ValueError):
        canonical_rotation(1, 12)
    with pytest.raises(ValueError):
        canonical_rotation(1, 1)


def test_compact_fits_rejects_bad_inputs():
    q0 = (1 << 60) - 131071
    assert not compact_plaintext_fits([float("nan")], 4, 2.0**40, q0)
    assert not compact_plaintext_fits([1.0], 4, float("inf"), q0)
    assert not compact_plaintext_fits([1.0], 4, -1.0, q0)
    assert not compact_plaintext_fits([1.0] * 5, 4, 2.0**40, q0)
    assert not compact_plaintext_fits([1.0], 4, 2.0**40, 3)
    assert not compact_plaintext_fits([1.0], 4, 2.0**40, 1 << 61)
    assert compact_plaintext_fits([], 4, 2.0**40, q0)


def _prefix_batch_run(offsets, slots, naf):
    """Values are rotation amounts; rotate adds, siblings adds per step."""
    log = []

    def rotate(v, step):
        log.append(("rot", v, step))
        return v + step

    def siblings(v, steps):
        log.append(("sib", v, tuple(steps)))
        return [v + s for s in steps]

    stats = RotationBatchStats()
    out = rotate_prefix_batch(0, offsets, slots, naf, rotate, siblings, stats)
    return out, stats, log


@pytest.mark.parametrize("naf", [False, True])
def test_prefix_batch_results_and_sharing(naf):
    slots = 256
    rng = random.Random(7)
    offsets = [rng.randrange(-600, 600) for _ in range(60)] + [0, 0, 1, 1]
    out, stats, log = _prefix_batch_run(offsets, slots, naf)
    for off, got in zip(offsets, out):
        assert got == canonical_rotation(off, slots)
        assert got == sum(rotation_steps(off, slots, naf))
    # every distinct step prefix is one tree edge
    prefixes = set()
    for off in offsets:
        steps = rotation_steps(off, slots, naf)
        for k in range(1, len(steps) + 1):
            prefixes.add(tuple(steps[:k]))
    assert stats.edges == len(prefixes)
    assert stats.requests == len(offsets)
    rot_edges = sum(1 for e in log if e[0] == "rot")
    sib_edges = sum(len(e[2]) for e in log if e[0] == "sib")
    assert rot_edges + sib_edges == stats.edges
    assert stats.preparations == len(log)
    assert stats.sibling_batches == sum(1 for e in log if e[0] == "sib")


def test_prefix_batch_visit_order_is_depth_first_ascending():
    # offsets 1, 2, 3 (binary): root children {1, 2}; child 1 has child 2.
    out, stats, log = _prefix_batch_run([3, 2, 1], 64, False)
    assert out == [3, 2, 1]
    assert log == [("sib", 0, (1, 2)), ("rot", 1, 2)]
    # the subtree under the smaller step is finished before the larger one
    out, _, log = _prefix_batch_run([5, 3, 6], 64, False)
    assert out == [5, 3, 6]
    assert log == [("sib", 0, (1, 2)), ("sib", 1, (2, 4)), ("rot", 2, 4)]


def test_prefix_batch_size_mismatch_raises():
    with pytest.raises(RuntimeError):
        rotate_prefix_batch(0, [1, 2], 64, False, lambda v, s: v + s,
                            lambda v, steps: [v], RotationBatchStats())
