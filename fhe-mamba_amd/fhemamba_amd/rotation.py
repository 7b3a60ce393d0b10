"""Rotation planning: signed-digit step decomposition and hoisted batching.

Restates the reference's rotation planner so the same key set serves the
same offsets:
  * naf_steps / canonical_rotation / rotation_steps follow
    native/fideslib_stage0/include/rotation_steps.hpp:11-47 (non-adjacent
    form, ascending magnitude; offsets folded into (-slots/2, slots/2]);
  * rotate_prefix_batch follows include/rotation_batch.hpp:17-62: outputs
    sharing a prefix of their step sequence share its rotations, and the
    children of one node are produced by one hoisted call;
  * bsgs_rotations lists the keys of a baby-step giant-step transform's
    hoisted schedule (CryptoContext.LinearTransformInPlace).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Sequence

INT_MIN, INT_MAX = -(2**31), 2**31 - 1


def naf_steps(value: int) -> list[int]:
    """Signed powers of two (non-adjacent form), smallest magnitude first."""
    steps: list[int] = []
    remaining, power = int(value), 1
    while remaining != 0:
        if remaining & 1:
            digit = 2 - (remaining & 3)  # +1 or -1
            step = digit * power
            if not INT_MIN <= step <= INT_MAX:
                raise OverflowError("NAF step exceeds signed rotation index")
            steps.append(step)
            remaining -= digit
        remaining //= 2  # exact: remaining is even here
        power *= 2
    return steps


def canonical_rotation(offset: int, slots: int) -> int:
    if slots < 2 or slots & (slots - 1):
        raise ValueError("rotation slots must be a power of two")
    offset = int(offset)
    # remainder with the dividend's sign, as C++ % computes it
    offset = -(-offset % slots) if offset < 0 else offset % slots
    if offset > slots // 2:
        offset -= slots
    if offset < -(slots // 2):
        offset += slots
    return offset


def rotation_steps(offset: int, slots: int, naf: bool) -> list[int]:
    offset = canonical_rotation(offset, slots)
    if naf:
        return naf_steps(offset)
    sign = -1 if offset < 0 else 1
    steps, bits, power = [], abs(offset), 1
    while bits:
        if bits & 1:
            steps.append(sign * power)
        bits >>= 1
        power <<= 1
    return steps


@dataclass
class RotationBatchStats:
    requests: int = 0
    edges: int = 0
    preparations: int = 0
    sibling_batches: int = 0


def rotate_prefix_batch(value, offsets: Sequence[int], slots: int, naf: bool,
                        rotate: Callable, siblings: Callable,
                        stats: RotationBatchStats | None = None) -> list:
    """Rotate `value` by every offset, sharing identical step prefixes.

    rotate(v, step) -> rotated value; siblings(v, steps) -> list of rotated
    values (one hoisted precompute for all steps)."""
    stats = stats if stats is not None else RotationBatchStats()
    children: list[dict[int, int]] = [{}]
    outputs: list[list[int]] = [[]]
    for i, off in enumerate(offsets):
        node = 0
        for step in rotation_steps(off, slots, naf):
            nxt = children[node].get(step)
            if nxt is None:
                nxt = len(children)
                children[node][step] = nxt
                children.append({})
                outputs.append([])
            node = nxt
        outputs[node].append(i)
    stats.requests += len(offsets)
    results: list = [None] * len(offsets)
    # Depth-first, children in ascending step order (the reference recurses
    # over a std::map), so callbacks run in the reference's order.
    stack = [(0, value)]
    while stack:
        node, val = stack.pop()
        for out in outputs[node]:
            results[out] = val
        kids = sorted(children[node].items())
        if not kids:
            continue
        stats.preparations += 1
        stats.edges += len(kids)
        if len(kids) == 1:
            step, child = kids[0]
            stack.append((child, rotate(val, step)))
        else:
            stats.sibling_batches += 1
            steps = [s for s, _ in kids]
            vals = list(siblings(val, steps))
            if len(vals) != len(steps):
                raise RuntimeError("rotation batch size mismatch")
            for (_, child), v in reversed(list(zip(kids, vals))):
                stack.append((child, v))
    return results


def bsgs_rotations(count: int, bstep: int, stride: int, offset: int = 0,
                   used=None) -> list[int]:
    """Rotation indices whose keys give LinearTransformInPlace its fast
    schedule for `count` diagonals at `stride` from `offset`: the babies
    offset + b*stride (b in `used`, default every baby; b = 0 only with an
    offset) and every giant multiple g*bstep*stride."""
    nb = min(bstep, count)
    used = range(nb) if used is None else used
    out = [offset + b * stride for b in used if b or offset]
    out += [g * bstep * stride for g in range(1, -(-count // bstep))]
    return out
