"""bench.py's operation tally for the decode CPU estimate (OpTally), on a
stand-in device context: every wrapped call is counted by class and limb
count, linear transforms break down into their ModUp, hoisted baby key
switches, giant-step key switches and diagonal products, and leaving the
block restores the methods."""
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import bench  # noqa: E402


class P:
    def __init__(self, nlimb):
        self.nlimb = nlimb


class Ctx:
    def _r(self, *a, **k):
        return "done"

    add = sub = negate = add_plain = add_const = _r
    mul_plain = mul_const = mul_int = _r
    keyswitch = relinearize = rotate = rescale = tensor = rotation_precompute = _r
    mod_raise = linear_wsum = rotate_hoisted = rotate_many = _r
    relinearize_many = rescale_many = _r
    linear_transform = linear_transform_hoisted = encode = encode_many = _r


def test_tally_counts_and_restores():
    originals = {k: v for k, v in vars(Ctx).items() if not k.startswith("__")}
    c = Ctx()
    with bench.OpTally(Ctx) as t:
        assert c.add(P(10), P(10)) == "done"
        c.negate(P(10))
        c.mul_plain(P(7), P(7))
        c.rotate(P(12), None, 5)
        c.relinearize(P(12), None)
        c.rescale(P(12))
        c.rotate_hoisted(P(9), None, [1, 2, 3], [5, 25, 125])
        c.rotate_many([P(8), P(8)], [1, 2], [5, 25])
        c.mod_raise(P(1), 30)
        c.linear_wsum([P(6)] * 4, [1, 2, 3, 4], 5)
        # 10 diagonals (2 zero), baby step 4: 3 giants, babies 1..3 rotated
        c.linear_transform_hoisted(P(20), [1] * 8 + [None] * 2, 4, [None, 1, 2, 3], [1, 5, 25, 125],
                                   giant_keys=[1, 2], giant_galois=[7, 49])
        c.encode_many([[0.0]] * 5, 8, 2.0**40, 3)
        c.relinearize_many([P(11)] * 3, None)
        c.rescale_many([P(11)] * 4)
        snap = t.snapshot()
    assert snap == {("add", 10): 2, ("pmul", 7): 1, ("ks", 12): 2, ("rescale", 12): 1,
                    ("hks", 9): 3, ("ks", 8): 2, ("modraise", 30): 1, ("pmul", 5): 4,
                    ("pmul", 20): 8, ("modup", 20): 1, ("hks", 20): 3, ("ks", 20): 2,
                    ("encode", 3): 5, ("ks", 11): 3, ("rescale", 11): 4}
    assert {k: v for k, v in vars(Ctx).items() if not k.startswith("__")} == originals
