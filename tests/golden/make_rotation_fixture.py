"""Record the reference planner's step decompositions as a fixture.

Runs oracle/_ref/ref_headers (built by `make -C oracle ref` from the
reference's native/fideslib_stage0/include/rotation_steps.hpp and
plaintext_rns.hpp) over a grid of offsets and bound cases and writes
tests/golden/rotation_steps.json.  Run where the reference tree is mounted;
the fixture is committed.
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))

import oracle as O  # noqa: E402


def main() -> int:
    if not O.ref_driver_available():
        print("reference driver not built (make -C oracle ref)", file=sys.stderr)
        return 1
    nafs = list(range(-300, 301)) + [1 << 20, -(1 << 20) + 3, 2**31 - 1, -(2**31) + 1]
    rots = [(off, slots, naf) for slots in (2, 8, 64, 32768) for naf in (0, 1)
            for off in (-70000, -32768, -16385, -100, -33, -17, -1, 0, 1, 5, 17, 33, 100, 16384,
                        16385, 32767, 32768, 70001)]
    fits = [
        (2, 2.0**59, (1 << 60) - 131071, [0.0, -0.0]),
        (2, 2.0**59, (1 << 60) - 131071, [0.49, -0.49]),
        (2, 2.0**59, (1 << 60) - 131071, [0.51, -0.51]),
        (2, 2.0**59, (1 << 60) - 131071, [1.0, -1.0]),
        (4, 2.0**59, (1 << 60) - 131071, [1.0]),
        (1, 2.0**59, (1 << 60) - 131071, [0.0, 0.0]),
        (8, 2.0**40, (1 << 50) - 1, [0.25, -3.0, 7.5]),
        (8, 2.0**40, (1 << 50) - 1, [1000.0, -3.0, 7.5]),
    ]
    lines = [f"naf {v}" for v in nafs]
    lines += [f"rot {o} {s} {n}" for o, s, n in rots]
    lines += ["fits %d %r %d %s" % (s, sc, q, " ".join(repr(v) for v in vals))
              for s, sc, q, vals in fits]
    out = O.ref_driver(lines)
    parse = lambda t: None if t.strip() == "error" else [int(x) for x in t.split()]  # noqa: E731
    fixture = {
        "source": "native/fideslib_stage0/include/rotation_steps.hpp, plaintext_rns.hpp",
        "naf": [[v, parse(out[i])] for i, v in enumerate(nafs)],
        "rotation_steps": [[o, s, n, parse(out[len(nafs) + i])] for i, (o, s, n) in enumerate(rots)],
        "compact_fits": [[s, sc, q, vals, int(out[len(nafs) + len(rots) + i])]
                         for i, (s, sc, q, vals) in enumerate(fits)],
    }
    with open(os.path.join(HERE, "rotation_steps.json"), "w") as fh:
        json.dump(fixture, fh)
        fh.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
