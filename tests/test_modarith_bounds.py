"""The lazy-reduction bounds that bit-exactness rests on, checked on the CPU.

fhe-mamba_amd/csrc/modarith.hpp is compiled for the host (tests/
modarith_driver.cpp: the kernels' own helpers, and the NTT butterflies
composed from them as the kernels compose them) and every result is
checked with unbounded integers: the congruence and the stated output range,
on random inputs across the stated input range and on inputs at its edges
(0, the largest allowed value, both ends of the modulus range).  This is the
method of the reference's experiments/ntt_lazy/check_arithmetic.py (integer
identity and range of the lazy butterfly), applied to each helper.

Moduli: odd values at both ends of each helper's range.  The plain NTT
passes take q < 2^61 (8q < 2^64); the fused ModDown passes and reduce_est
take q in [2^33, 2^60) (16q < 2^64, and the float quotient estimate needs
q >= 2^33).  Primality plays no part in these identities."""
import os
import random
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "fhe-mamba_amd", "csrc")
M64 = (1 << 64) - 1
R64 = 1 << 64

Q_PLAIN = [(1 << 33) + 1, (1 << 40) + 15, (1 << 50) + 55, (1 << 59) - 55, (1 << 60) - 93,
           (1 << 60) + 33, (1 << 61) - 1]
Q_FUSED = [q for q in Q_PLAIN if q < (1 << 60)] + [(1 << 60) - 1]
N_RANDOM = 4000


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = str(tmp_path_factory.mktemp("modarith") / "modarith_driver")
    cmd = [cxx, "-std=c++17", "-O2", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I" + CSRC, os.path.join(HERE, "modarith_driver.cpp"), "-o", exe]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip("modarith.hpp does not build for the host here:\n" + res.stderr[-2000:])
    return exe


def run(exe, op, records, nout):
    data = np.asarray(records, dtype=np.uint64).tobytes()
    res = subprocess.run([exe, op], input=data, capture_output=True, check=True)
    out = np.frombuffer(res.stdout, dtype=np.uint64).reshape(len(records), nout)
    return [[int(v) for v in row] for row in out]


def edge_and_random(rng, hi, edges):
    """Edge values below hi, then random ones."""
    vals = [v for v in edges if 0 <= v < hi]
    return vals + [rng.randrange(hi) for _ in range(N_RANDOM)]


@pytest.mark.parametrize("op,bound", [("shoup_lazy", 2), ("shoup_lazy4", 4), ("shoup_lazy4n", 4)])
def test_shoup_products(driver, op, bound):
    """a * w mod q for any 64-bit a and w < q: [0, 2q) exact quotient,
    [0, 4q) approximate quotient (three 32x32 partial products)."""
    rng = random.Random(11)
    recs = []
    for q in Q_PLAIN:
        ws = [0, 1, q - 1, (q - 1) // 2] + [rng.randrange(q) for _ in range(40)]
        a_vals = edge_and_random(rng, R64, [0, 1, q - 1, q, 4 * q - 1, 8 * q - 1, M64,
                                            M64 - q, 1 << 63, (1 << 32) - 1, 1 << 32])
        for i, a in enumerate(a_vals):
            recs.append((q, a, ws[i % len(ws)]))
    out = run(driver, op, recs, 1)
    for (q, a, w), (r,) in zip(recs, out):
        assert 0 <= r < bound * q, (op, q, a, w, r)
        assert r % q == a * w % q, (op, q, a, w, r)


def test_lazy_sub(driver):
    """x >= m ? x - m : x for m <= 2^63 and x - m < 2^63 when x >= m; m is
    4q or 8q in the kernels."""
    rng = random.Random(12)
    recs = []
    for q in Q_PLAIN:
        for m in (4 * q, 8 * q):
            if m > 1 << 63:
                continue
            top = min(m + (1 << 63) - 1, M64)  # x - m < 2^63
            xs = edge_and_random(rng, top + 1, [0, 1, m - 1, m, m + 1, 2 * m - 1, top])
            recs += [(q, x, m) for x in xs]
    out = run(driver, "lazy_sub", recs, 1)
    for (q, x, m), (r,) in zip(recs, out):
        assert r == (x - m if x >= m else x), (q, x, m, r)


def test_redc(driver):
    """T 2^-64 mod q in [0, q) for T = hi 2^64 + lo < q 2^64."""
    rng = random.Random(13)
    recs = []
    for q in Q_PLAIN:
        his = edge_and_random(rng, q, [0, 1, q - 1])
        for i, hi in enumerate(his):
            lo = [0, 1, M64, rng.randrange(R64)][i % 4]
            recs.append((q, hi, lo))
    out = run(driver, "redc", recs, 1)
    for (q, hi, lo), (r,) in zip(recs, out):
        t = hi * R64 + lo
        assert 0 <= r < q and r == t * pow(R64, -1, q) % q, (q, hi, lo, r)


def test_redc_lazy(driver):
    """Montgomery reduction without the final correction: (0, 2q) for hi < q."""
    rng = random.Random(14)
    recs = []
    for q in Q_PLAIN:
        his = edge_and_random(rng, q, [0, 1, q - 1])
        for i, hi in enumerate(his):
            lo = [0, 1, M64, rng.randrange(R64)][i % 4]
            recs.append((q, hi, lo))
    out = run(driver, "redc_lazy", recs, 1)
    for (q, hi, lo), (r,) in zip(recs, out):
        t = hi * R64 + lo
        assert 0 < r < 2 * q and r % q == t * pow(R64, -1, q) % q, (q, hi, lo, r)


def test_reduce_est(driver):
    """x mod q for x < 2^18 q (and below 2^64), q in [2^33, 2^60]: quotient
    estimate from a float, at most one low, one conditional subtraction."""
    rng = random.Random(15)
    recs = []
    for q in Q_FUSED:
        top = min((1 << 18) * q, R64)  # x is a 64-bit word
        edges = [0, 1, q - 1, q, q + 1, 2 * q - 1, 15 * q - 1, 15 * q, top - 1, top - q,
                 top - q - 1] + [k * q + d for k in (1 << 17, (1 << 18) - 1, 12345)
                                 for d in (-1, 0, 1) if 0 <= k * q + d < top]
        recs += [(q, x) for x in edge_and_random(rng, top, edges)]
    out = run(driver, "reduce_est", recs, 1)
    for (q, x), (r,) in zip(recs, out):
        assert r == x % q, (q, x, r)


def butterfly_cases(rng, qs, in_bound):
    recs = []
    for q in qs:
        top = in_bound * q
        ws = [0, 1, q - 1] + [rng.randrange(q) for _ in range(30)]
        edges = [0, 1, q - 1, 4 * q - 1, top - 1]
        xs = edge_and_random(rng, top, edges)
        for i, x in enumerate(xs):
            y = edges[i % len(edges)] if i < 25 else rng.randrange(top)
            recs.append((q, x, y, ws[i % len(ws)]))
    return recs


def test_forward_butterfly(driver):
    """Plain forward stage: inputs below 8q stay below 8q (q < 2^61)."""
    recs = butterfly_cases(random.Random(16), Q_PLAIN, 8)
    out = run(driver, "fwd", recs, 2)
    for (q, x, y, w), (u, v) in zip(recs, out):
        assert u < 8 * q and v < 8 * q, (q, x, y, w, u, v)
        assert u % q == (x + y * w) % q and v % q == (x - y * w) % q


def test_inverse_butterfly(driver):
    """Inverse stage: inputs below 4q stay below 4q."""
    recs = butterfly_cases(random.Random(17), Q_PLAIN, 4)
    out = run(driver, "inv", recs, 2)
    for (q, x, y, w), (u, v) in zip(recs, out):
        assert u < 4 * q and v < 4 * q, (q, x, y, w, u, v)
        assert u % q == (x + y) % q and v % q == (x - y) * w % q


def test_alternating_forward_range(driver):
    """The fused ModDown's alternating range (q < 2^60): a stage that first
    brings X below 8q takes inputs below 16q and leaves them below 12q; the
    next stage adds without reducing and leaves them below 16q; the sum the
    epilogue reduces (last stage < 12q, key sum < 2q, addend < q) is below
    15q, inside reduce_est's 2^18 q."""
    rng = random.Random(18)
    even = butterfly_cases(rng, Q_FUSED, 16)
    out = run(driver, "fwd_alt_even", even, 2)
    for (q, x, y, w), (u, v) in zip(even, out):
        assert u < 12 * q and v < 12 * q, (q, x, y, w, u, v)
        assert u % q == (x + y * w) % q and v % q == (x - y * w) % q
    odd = butterfly_cases(rng, Q_FUSED, 12)
    out = run(driver, "fwd_alt_odd", odd, 2)
    for (q, x, y, w), (u, v) in zip(odd, out):
        assert u < 16 * q and v < 16 * q, (q, x, y, w, u, v)
        assert u % q == (x + y * w) % q and v % q == (x - y * w) % q


def test_a_planted_range_error_is_caught(driver):
    """The range checks are live: a plain forward stage fed inputs above its
    stated bound (below 16q instead of 8q) leaves the 8q range."""
    recs = [(q, 16 * q - 1, 16 * q - 1, q - 1) for q in Q_PLAIN if 16 * q < R64]
    out = run(driver, "fwd", recs, 2)
    assert any(u >= 8 * q or v >= 8 * q for (q, *_), (u, v) in zip(recs, out))
