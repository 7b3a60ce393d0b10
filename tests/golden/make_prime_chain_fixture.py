"""Extract the OpenFHE prime chain recorded by the reference into a fixture.

Reads results/b300/2026-09-28/long-accuracy/oracle-p-r3-base/native.json
(`all_primes`: 45 Q primes then 12 P primes of the OpenFHE 1.4.2 context
N=2^17, depth 44, scaling mod size 59, first mod size 60, dnum 4, built by
experiments/ntt_warp_tail/probe.cu:97-103) and writes
tests/golden/openfhe_prime_chain_n131072.json.  Run only where the
reference tree is mounted; the fixture is committed.
"""
import json
import os
import sys

REFERENCE = os.environ.get("FHEMAMBA_REFERENCE", "/root/reference")
SRC = "results/b300/2026-09-28/long-accuracy/oracle-p-r3-base/native.json"


def main() -> int:
    with open(os.path.join(REFERENCE, SRC)) as fh:
        record = json.load(fh)
    primes = [int(p) for p in record["all_primes"]]
    fixture = {
        "source": SRC,
        "ring_dimension": int(record["ring"]),
        "multiplicative_depth": 44,
        "scaling_mod_size": 59,
        "first_mod_size": 60,
        "num_large_digits": int(record["digits"]),
        "num_q": 45,
        "num_p": len(primes) - 45,
        "primes": primes,
    }
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                       "openfhe_prime_chain_n131072.json")
    with open(out, "w") as fh:
        json.dump(fixture, fh, indent=1)
        fh.write("\n")
    print(out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
