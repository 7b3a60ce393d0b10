"""Packed-program executor on the CPU: the reader against the reference's
own parser cases (native/fideslib_stage0/tests/test_packed_program.cpp),
output errors, the rotation-sum schedule, the replicated matrix layout and
monotone routing against numpy, and every node kind through the executor
on a slot-level stand-in for the CKKS context."""
import math

import numpy as np
import pytest

from fhemamba_amd import packed as P
from packed_builder import ProgramBuilder, SlotContext, SlotKeys

VALID = "fhemamba-packed-v1 8 64 2 1\ninput 2 0 2 1 2\ngather 2 1 0 2 1 0\n1 2 2 1 2 1\n"
EXTENDED = ("fhemamba-packed-v2 8 64 4 1\n"
            "input 2 8 0 2 1 2\nlinear 2 16 1 0 4 1 0 0 1\n"
            "linear_ref 2 16 1 0 1 1\nfeedback 2 8 1 2 0\n2 2 1 2 1 2\n")


def test_reader_accepts_the_reference_cases():
    p = P.read_packed_program(VALID)
    assert p.slots == 8 and len(p.nodes) == 2 and p.outputs[0].exact[0] == 2
    e = P.packed_output_errors([2.0005, 1], p.outputs[0])
    assert e.passes(.001, .001) and not e.passes(.0001, .001) and not e.passes(.001, .0001)
    assert not e.passes(math.inf, .001)
    nf = P.packed_output_errors([math.nan, 1], p.outputs[0])
    assert nf.non_finite == 1 and not nf.passes(.001, .001)
    with pytest.raises(ValueError):
        P.packed_output_errors([2], p.outputs[0])
    v2 = P.read_packed_program(EXTENDED)
    assert v2.nodes[2].operation == "linear_ref" and v2.nodes[2].bound == 16
    assert v2.nodes[3].operation == "feedback" and len(v2.nodes[3].data) == 0


def test_reader_parses_a_long_chain():
    n = 20000
    lines = [f"fhemamba-packed-v2 8 64 {n} 1", "input 1 8 0 1 1"]
    lines += [f"addp 1 8 1 {i - 1} 1 0" for i in range(1, n)]
    lines.append(f"{n - 1} 1 1 1")
    p = P.read_packed_program("\n".join(lines))
    assert len(p.nodes) == n and p.outputs[0].node == n - 1


@pytest.mark.parametrize("text", [
    "fhemamba-packed-v1 3 64 1 1",                                   # non-power-of-two slots
    "fhemamba-packed-v2 8 64 1000001 1",                             # node count bound
    "fhemamba-packed-v1 8 64 1 1 input 2 0 2 1 nan",                 # invalid constant
    "fhemamba-packed-v1 8 64 1 1 add 2 2 0 0 0",                     # future dependency
    "fhemamba-packed-v1 8 64 2 1 input 2 0 2 1 2 gather 1 1 0 1 2",  # index overflow
    VALID + "trailing",
    "fhemamba-packed-v2 8 64 1 1 input 2 65 0 2 1 2",                # bound above the header's
    "fhemamba-packed-v2 8 64 2 1 input 2 8 0 2 1 2 linear_ref 2 8 1 0 1 0",  # not a weight
    "fhemamba-packed-v2 8 64 2 1 input 2 8 0 2 1 2 feedback 3 8 1 0 0",      # width change
    "fhemamba-packed-v1 8 64 2 1 input 2 0 2 1 2 feedback 2 1 0 0",  # v2-only operation
    "fhemamba-packed-v1 8 64 2 1 input 4 0 4 1 2 3 4 repeat 12 1 0 3 1 4 3",  # v1 repeat 3
    "fhemamba-packed-v1 8 64 2 1 input 4 0 4 1 2 3 4 sum 1 1 0 1 3",  # width not 2^k
    "fhemamba-packed-v1 8 64 2 1 input 2 0 2 1 2 scatter 4 1 0 2 1 1",  # repeated target
    "fhemamba-packed-v1 8 64 2 1 input 2 0 2 1 2 cheb 2 1 0 4 1 0 1 1",  # lo >= hi
])
def test_reader_rejects(text):
    with pytest.raises(ValueError):
        P.read_packed_program(text)


@pytest.mark.parametrize("count", list(range(1, 41)) + [127, 128, 1000])
def test_rotation_sum_schedule_covers_every_shift_once(count):
    terms = {0: 1}       # shift -> multiplicity in the running sum
    for off, acc in P.rotation_sum_schedule(count):
        src = dict(terms) if acc else {0: 1}
        for k, c in src.items():
            terms[k + off] = terms.get(k + off, 0) + c
    assert terms == {k: 1 for k in range(count)}


def replicated_numpy(W, x, slots):
    """The replicated layout evaluated with numpy rotations."""
    m, n = W.shape
    s = P.replicated_shape(m, n, slots)
    rot = lambda v, k: np.roll(v, -k)  # noqa: E731
    v = np.zeros(slots)
    v[:n] = x

    def rsum(a, count, stride):
        out = a
        for off, acc in P.rotation_sum_schedule(count):
            out = out + rot(out if acc else a, off * stride)
        return out

    rep = rsum(rsum(v, s.reps, -n), s.replicas + s.guard, -s.window)
    out = np.zeros(slots)
    for k in range(s.per_replica):
        out += P.replicated_mask(W, k, s, slots) * rot(rep, k * s.replicas)
    out = rsum(out, s.replicas, s.window + 1)
    return out[:m], s


@pytest.mark.parametrize("m,n,slots", [(4, 4, 64), (8, 3, 64), (16, 24, 256), (48, 24, 1024),
                                       (100, 7, 1024), (1536, 768, 32768)])
def test_replicated_layout_computes_the_product(m, n, slots):
    rng = np.random.default_rng(m * n)
    W = rng.normal(size=(m, n))
    x = rng.normal(size=n)
    got, s = replicated_numpy(W, x, slots)
    assert s.replicas > 1
    assert (s.replicas + s.guard) * s.window <= slots and s.window % n == 0
    assert np.allclose(got, W @ x)


def test_replicated_shape_falls_back_when_nothing_fits():
    assert P.replicated_shape(60, 60, 64).replicas == 1
    s = P.replicated_shape(1536, 768, 32768)
    assert (s.replicas, s.window, s.per_replica) == (13, 2304, 60)


def route_numpy(x, idx, scatter, slots):
    rot = lambda v, k: np.roll(v, -k)  # noqa: E731
    v = np.zeros(slots)
    v[: len(x)] = x
    for stage in P.monotone_routing(idx, scatter):
        nxt = np.zeros(slots)
        for off, positions in stage.items():
            sel = np.zeros(slots)
            sel[positions] = 1
            nxt += rot(v * sel, off)
        v = nxt
    return v


def test_monotone_routing_gathers_and_scatters():
    rng = np.random.default_rng(3)
    slots = 4096
    idx = np.sort(rng.choice(3000, 200, replace=False))
    x = rng.normal(size=3000)
    g = route_numpy(x, idx, False, slots)
    assert np.allclose(g[:200], x[idx]) and np.allclose(g[200:], 0)
    y = rng.normal(size=200)
    sc = route_numpy(y, idx, True, slots)
    want = np.zeros(slots)
    want[idx] = y
    assert np.allclose(sc, want)
    with pytest.raises(ValueError):
        P.monotone_routing([3, 2], False)


# ---------------------------------------------------------------- executor
def run_slots(builder, **kw):
    program = P.read_packed_program(builder.text())
    cc = SlotContext(program.slots)
    ev = P.PackedEvaluator(cc, SlotKeys(), program.slots, **kw)
    outs = ev.evaluate(program)
    return program, ev, [ev.decrypt(ct, len(o.polynomial)) for o, ct in zip(program.outputs, outs)]


def check(builder, tol=1e-9, **kw):
    program, ev, values = run_slots(builder, **kw)
    for o, v in zip(program.outputs, values):
        e = P.packed_output_errors(v, o)
        assert e.passes(tol, tol), (e, o.node, program.nodes[o.node].operation)
    return ev


def test_every_node_kind_on_slots():
    rng = np.random.default_rng(5)
    b = ProgramBuilder(256, bound=64.0, extended=True)
    x = b.input(rng.uniform(-1, 1, 16))
    c = b.public(rng.uniform(-1, 1, 16))
    s = b.add(x, c)
    m = b.mul(s, x)
    sq = b.mul(m, m)
    ap = b.addp(sq, rng.uniform(-1, 1, 16))
    mp = b.mulp(ap, rng.uniform(-1, 1, 16))
    W = rng.normal(size=(24, 16)) * 0.3
    lin = b.linear(mp, W)
    lr = b.linear_ref(x, lin)                  # shared weight table
    g = b.gather(lin, [3, 1, 4, 1, 5, 9, 2, 6])   # non-monotone
    sc = b.scatter(g, [0, 2, 4, 6, 8, 10, 12, 14], 16)
    rp = b.repeat(sc, 2, 8, 3)
    sm = b.sum(b.addp(rp, np.zeros(48)), 16)
    ch = b.cheb(x, -1.5, 1.5, [0.1, 0.5, -0.2, 0.05, 0.01, -0.003])
    for node in (s, m, sq, ap, mp, lin, lr, g, sc, rp, sm, ch):
        b.output(node)
    ev = check(b)
    assert ev.stats["rotations"] > 0 and ev.stats["logical_refreshes"] == 0


def test_direct_linear_matches_replicated():
    rng = np.random.default_rng(6)
    b = ProgramBuilder(512)
    x = b.input(rng.uniform(-1, 1, 32))
    b.output(b.linear(x, rng.normal(size=(40, 32))))
    check(b, replicated_linear=False)
    check(b, replicated_linear=True)


def test_large_monotone_gather_uses_routing_stages():
    rng = np.random.default_rng(7)
    b = ProgramBuilder(4096)
    x = b.input(rng.uniform(-1, 1, 3000))
    idx = np.sort(rng.choice(3000, 300, replace=False))
    g = b.gather(x, idx)
    b.output(g)
    b.output(b.scatter(g, idx, 3000))
    check(b)


def test_deep_chain_is_refreshed():
    """120 levels of products pass the ceiling several times."""
    rng = np.random.default_rng(8)
    b = ProgramBuilder(64, bound=4.0)
    v = b.input(rng.uniform(0.5, 1.5, 8))
    w = b.input(np.ones(8))
    for _ in range(60):                     # v <- (v * w) * 1: two levels, same value,
        v = b.mulp(b.mul(v, w), np.ones(8))  # errors add (no amplification)
    b.output(v)
    program, ev, values = run_slots(b)
    assert ev.stats["logical_refreshes"] >= 3
    assert ev.stats["bootstraps"] == 2 * ev.stats["logical_refreshes"]
    assert np.allclose(values[0], b.values[v])


def test_feedback_uses_the_client():
    rng = np.random.default_rng(9)
    b = ProgramBuilder(64, extended=True)
    h = b.input(rng.uniform(-1, 1, 4))
    fb = b.feedback(h, np.zeros(4))
    b.output(h)
    b.output(fb, np.full(4, 7.0))
    program = P.read_packed_program(b.text())
    calls = []

    def client(ev, node, hidden):
        calls.append(node)
        return np.full(4, 7.0)

    ev = P.PackedEvaluator(SlotContext(64), SlotKeys(), 64, client=client)
    outs = ev.evaluate(program)
    assert calls == [1] and np.allclose(ev.decrypt(outs[1], 4), 7.0)
    with pytest.raises(RuntimeError):
        P.PackedEvaluator(SlotContext(64), SlotKeys(), 64).evaluate(program)


def test_command_line_options():
    o = P.parse_args(["p.txt", "r.json", "1e-3", "1e-2", "--bootstrap-passes", "1",
                      "--cache-plaintexts", "--prefetch-workers", "2", "--direct-linear"])
    assert o["bootstrap_passes"] == 1 and o["direct_linear"] and o["exact_tol"] == 1e-2
    assert o["accepted"] == ["--cache-plaintexts", "--prefetch-workers 2"]
    for bad in (["p", "r", "1"], ["p", "r", "0", "1"], ["p", "r", "1", "1", "--bogus"],
                ["p", "r", "1", "1", "--bootstrap-passes", "3"],
                ["p", "r", "1", "1", "--security", "256"],
                ["p", "r", "1", "1", "--security-digits", "3"],
                ["p", "r", "1", "1", "--security", "128-classic", "--security-digits", "0"],
                ["p", "r", "1", "1", "--security", "128-classic", "--security-digits", "17"],
                ["p", "r", "1", "1", "--s2c-first"],
                ["p", "r", "1", "1", "--s2c-first", "--batch-refresh"],
                ["p", "r", "1", "1", "--batch-refresh", "--planned-refresh",
                 "--bootstrap-passes", "1"],
                ["p", "r", "1", "1", "--gpu-dual-ring"]):
        with pytest.raises(ValueError):
            P.parse_args(bad)


def test_s2c_first_options():
    """--s2c-first needs planned two-pass batch refresh
    (packed_fideslib.cpp:1013-1017); it is recorded as its own option."""
    o = P.parse_args(["p", "r", "1e-3", "1e-2", "--planned-refresh", "--batch-refresh",
                      "--s2c-first"])
    assert o["s2c_first"] and o["accepted"] == ["--planned-refresh", "--batch-refresh"]
    with pytest.raises(ValueError, match="batch refresh"):
        P.parse_args(["p", "r", "1e-3", "1e-2", "--planned-refresh", "--s2c-first"])


def test_classical128_options():
    """--security 128-classic with the reference's digit rule: 4 digits by
    default, --security-digits 1..16 only with it (packed_fideslib.cpp:913,
    974, 991-992)."""
    o = P.parse_args(["p", "r", "1e-3", "1e-2", "--security", "128-classic"])
    assert o["security"] == "128-classic" and o["security_digits"] == 4
    o = P.parse_args(["p", "r", "1e-3", "1e-2", "--security", "128-classic",
                      "--security-digits", "6"])
    assert o["security_digits"] == 6 and o["accepted"] == []


def test_classical128_chain_passes_the_audit_at_n17_only():
    """The classical-128 chain the executor builds (depth 44, scale 59,
    first 60, 4 digits, uniform ternary) passes the audit at N=2^17 with the
    recorded QP of 3376 bits; the same depth at N=2^16 cannot (its bound is
    1747 bits), nor can a sparse-ternary secret."""
    from fhemamba_amd import ckks
    from fhemamba_amd.core import gen_moduli
    q, p = gen_moduli(17, 44, 59, 60, 4)
    a = ckks.audit_chain(131072, q, p, 4, security_level=ckks.SecurityLevel.HEStd_128_classic,
                         secret_dist=ckks.SecretKeyDist.UNIFORM_TERNARY)
    assert a["passed"] and a["qp_bits"] == 3376 and a["q_towers"] == 45 and a["p_towers"] == 12
    q16, p16 = gen_moduli(16, 44, 59, 60, 4)
    a16 = ckks.audit_chain(65536, q16, p16, 4,
                           security_level=ckks.SecurityLevel.HEStd_128_classic,
                           secret_dist=ckks.SecretKeyDist.UNIFORM_TERNARY)
    assert not a16["passed"] and a16["qp_bits"] > 1747


def test_client_head_reader(tmp_path):
    rng = np.random.default_rng(10)
    w = rng.normal(size=(5, 4)).astype("<f4")
    path = tmp_path / "head.f32"
    path.write_bytes(np.array([5, 4], dtype="<u4").tobytes() + w.tobytes())
    c = P.GenerationClient(str(path))
    h = rng.normal(size=4)
    emb = c.select(h)
    best = int(np.argmax(w.astype(np.float64) @ h))
    assert c.tokens == [best] and np.allclose(emb, w[best])
    path.write_bytes(np.array([5, 4], dtype="<u4").tobytes() + w.tobytes()[:-4])
    with pytest.raises(ValueError):
        P.GenerationClient(str(path))


def test_launcher_reports_bad_arguments_with_exit_code_2():
    import os
    import subprocess
    import sys
    launcher = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "fhe-mamba_amd", "packed_fhemamba")
    r = subprocess.run([sys.executable, launcher, "p.txt", "r.json", "1e-3"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "usage" in r.stderr


@pytest.mark.parametrize("free_gib, want", [(None, 48 << 30), (288, 96 << 30),
                                             (150, 54 << 30), (90, (90 << 30) // 8),
                                             (4, 512 << 20)])
def test_plaintext_cache_budget_follows_free_device_memory(monkeypatch, free_gib, want):
    """96 GiB (the 130M-shape decode's projection diagonals, ~53 GiB per
    token, fit), less when under 192 GiB are free, never below an eighth of
    the free memory (so never above it); 48 GiB when the free memory cannot
    be read.  The free memory is that of the device asked for."""
    from fhemamba_amd import _lib
    seen = []

    def free(device=None):
        seen.append(device)
        return None if free_gib is None else free_gib << 30
    monkeypatch.setattr(_lib, "device_free_bytes", free)
    assert P.default_pt_cache_bytes(3) == want
    assert seen == [3]


@pytest.mark.parametrize("count,support", [(2, 64), (5, 40), (6, None)])
def test_refresh_many_packs_pairs(count, support):
    """refresh_many under S2C-first on the slot-level stand-in: the values
    go in complex pairs, (a + i b) / 2 with the 1/2 on the support mask,
    one complex-slot bootstrap each (the odd one alone), and come back as
    the masked values themselves, at the bootstrap's output level; the
    ordinary order refreshes them one real bootstrap each."""
    slots = 64
    rng = np.random.default_rng(count)
    vals = [rng.uniform(-3, 3, slots) for _ in range(count)]
    for s2c_first in (True, False):
        cc = SlotContext(slots)
        ev = P.PackedEvaluator(cc, SlotKeys(), slots, s2c_first=s2c_first)
        cts = [ev.encrypt(v) for v in vals]
        sup = slots if support is None else support
        outs = ev.refresh_many(cts, 4.0, sup, passes=2)
        assert len(outs) == count
        want_calls = [(count + 1) // 2] if s2c_first else [count]
        assert cc.bootstrap_many_calls == want_calls
        assert ev.stats["bootstraps"] == 2 * want_calls[0]
        for v, o in zip(vals, outs):
            want = np.where(np.arange(slots) < sup, v, 0.0)
            assert np.allclose(o.z, want, atol=1e-12)
            assert o.GetLevel() == outs[0].GetLevel()
