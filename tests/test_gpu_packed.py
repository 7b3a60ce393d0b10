"""Packed-program executor on the GPU: programs written in the
fhemamba-packed format run through the evaluator on a real CKKS context,
outputs decrypted and compared with the programs' own references (the
reference executor's pass criterion, packed_fideslib.cpp:1206-1222), and the
command line end to end with the report the reference's benchmark gates on
(src/fhemamba/benchmarks/packed.py:196-214).  Tolerance 1e-5 on values of
magnitude <= 4 (59-bit scale; refreshed values carry the two-pass
bootstrap's ~2^-30)."""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = pytest.importorskip("fhemamba_amd")
from fhemamba_amd import packed as P  # noqa: E402
from packed_builder import ProgramBuilder  # noqa: E402

TOL = 1e-5


def evaluate(builder, ring_dim=1 << 12, **kw):
    program = P.read_packed_program(builder.text())
    cc, keys = P.build_context(program.slots, ring_dim=ring_dim, seed=3)
    ev = P.PackedEvaluator(cc, keys, program.slots, **kw)
    outs = ev.evaluate(program)
    errs = [P.packed_output_errors(ev.decrypt(ct, len(o.polynomial)), o)
            for o, ct in zip(program.outputs, outs)]
    return ev, errs


def test_every_node_kind():
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
    lr = b.linear_ref(x, lin)
    g = b.gather(lin, [3, 1, 4, 1, 5, 9, 2, 6])
    sc = b.scatter(g, [0, 2, 4, 6, 8, 10, 12, 14], 16)
    rp = b.repeat(sc, 2, 8, 3)
    sm = b.sum(b.addp(rp, np.zeros(48)), 16)
    ch = b.cheb(x, -1.5, 1.5, [0.1, 0.5, -0.2, 0.05, 0.01, -0.003])
    for node in (s, m, sq, ap, mp, lin, lr, g, sc, rp, sm, ch):
        b.output(node)
    ev, errs = evaluate(b)
    worst = max(e.polynomial for e in errs)
    print(f"all node kinds: max error {worst:.2e}, rotations {ev.stats['rotations']}",
          flush=True)
    assert all(e.passes(TOL, TOL) for e in errs), errs


def test_monotone_routing_and_direct_linear():
    rng = np.random.default_rng(7)
    b = ProgramBuilder(1024)
    x = b.input(rng.uniform(-1, 1, 800))
    idx = np.sort(rng.choice(800, 100, replace=False))
    g = b.gather(x, idx)
    b.output(g)
    b.output(b.scatter(g, idx, 800))
    b.output(b.linear(g, rng.normal(size=(30, 100)) * 0.1))
    for replicated in (True, False):
        ev, errs = evaluate(b, replicated_linear=replicated)
        assert all(e.passes(TOL, TOL) for e in errs), (replicated, errs)


def test_deep_chain_refreshes():
    rng = np.random.default_rng(8)
    b = ProgramBuilder(64, bound=4.0)
    v = b.input(rng.uniform(0.5, 1.5, 8))
    w = b.input(np.ones(8))
    for _ in range(60):                     # v <- (v * w) * 1: two levels, same value,
        v = b.mulp(b.mul(v, w), np.ones(8))  # errors add (no amplification)
    b.output(v)
    ev, errs = evaluate(b)
    print(f"deep chain: {ev.stats['logical_refreshes']} refreshes, error "
          f"{errs[0].polynomial:.2e}", flush=True)
    assert ev.stats["logical_refreshes"] >= 3
    assert errs[0].passes(TOL, TOL)


def test_command_line_report(tmp_path):
    """The reference's argv and parameters (N = 2^16, depth 44, scale 2^59)."""
    rng = np.random.default_rng(9)
    b = ProgramBuilder(512, bound=16.0, extended=True)
    x = b.input(rng.uniform(-1, 1, 64))
    h = b.cheb(b.linear(x, rng.normal(size=(64, 64)) * 0.1), -4, 4,
               [0.0, 0.6, 0.0, -0.05, 0.0, 0.002])
    b.output(b.sum(b.mul(h, h), 64), )
    prog, res = tmp_path / "program.txt", tmp_path / "native.json"
    prog.write_text(b.text())
    rc = P.main([str(prog), str(res), str(TOL), str(TOL), "--cache-plaintexts"])
    report = json.loads(res.read_text())
    assert rc == 0 and report["passed"] is True
    assert report["schema"] == "fhemamba-packed-result-v1" and report["encrypted"] is True
    assert report["non_finite"] == 0 and len(report["per_output_errors"]) == 1
    assert report["ring_dimension"] == 65536 and report["depth"] == 44
    assert report["diagnostic_only"] is False
    assert report["accepted_options"] == ["--cache-plaintexts"]
    # a program whose reference is wrong fails with exit code 1
    bad = b.text().splitlines()
    last = bad[-1].split()
    last[2] = str(float(last[2]) + 1.0)
    prog.write_text("\n".join(bad[:-1] + [" ".join(last)]) + "\n")
    assert P.main([str(prog), str(res), str(TOL), str(TOL)]) == 1
    assert json.loads(res.read_text())["passed"] is False


def test_command_line_classical128(tmp_path):
    """--security 128-classic as the reference executor runs it
    (packed_fideslib.cpp:1040-1075): ring 2^17, full packing (65536 slots),
    four HYBRID digits, uniform ternary, the audit written beside the
    report (RESULT.parameters.json) and in it; a deep enough program to
    refresh by full-packing bootstrapping at N=2^17."""
    rng = np.random.default_rng(12)
    b = ProgramBuilder(256, bound=4.0)
    v = b.input(rng.uniform(0.5, 1.5, 16))
    w = b.input(np.ones(16))
    for _ in range(30):
        v = b.mulp(b.mul(v, w), np.ones(16))
    b.output(v)
    prog, res = tmp_path / "program.txt", tmp_path / "native.json"
    prog.write_text(b.text())
    rc = P.main([str(prog), str(res), str(TOL), str(TOL), "--security", "128-classic"])
    report = json.loads(res.read_text())
    audit = json.loads((tmp_path / "native.json.parameters.json").read_text())
    print(f"classical-128 packed: eval {report['eval_seconds']:.2f}s, "
          f"{report['bootstraps']} bootstraps, error {report['max_abs_error_vs_polynomial']:.2e}",
          flush=True)
    assert rc == 0 and report["passed"] is True and report["security"] == "128-classic"
    assert report["ring_dimension"] == 131072 and report["slots"] == 65536
    assert report["security_audit"] == audit and audit["passed"] is True
    assert (audit["qp_bits"], audit["hybrid_digits"], audit["guideline_max_qp_bits"]) == \
        (3376, 4, 3523)
    assert report["logical_refreshes"] >= 1


def test_command_line_s2c_first(tmp_path):
    """--planned-refresh --batch-refresh --s2c-first (packed_fideslib.cpp:
    1013-1017, 1084-1086, 1131-1134): full packing at N = 2^16, refreshes by
    the SlotToCoeff-first bootstrap under a ceiling four levels lower, and
    the outputs within tolerance; a program that is not fully packed is
    refused."""
    rng = np.random.default_rng(13)
    b = ProgramBuilder(32768, bound=4.0)
    v = b.input(rng.uniform(0.5, 1.5, 64))
    w = b.input(np.ones(64))
    for _ in range(30):
        v = b.mulp(b.mul(v, w), np.ones(64))
    b.output(v)
    prog, res = tmp_path / "program.txt", tmp_path / "native.json"
    prog.write_text(b.text())
    flags = ["--planned-refresh", "--batch-refresh", "--s2c-first"]
    rc = P.main([str(prog), str(res), str(TOL), str(TOL)] + flags)
    report = json.loads(res.read_text())
    print(f"S2C-first packed: eval {report['eval_seconds']:.2f}s, {report['bootstraps']} "
          f"bootstraps, error {report['max_abs_error_vs_polynomial']:.2e}", flush=True)
    assert rc == 0 and report["passed"] is True and report["s2c_first"] is True
    assert report["refresh_ceiling"] == 45 - 3 - 4 and report["logical_refreshes"] >= 1
    small = ProgramBuilder(1024)
    small.output(small.input(np.ones(4)))
    prog.write_text(small.text())
    assert P.main([str(prog), str(res), str(TOL), str(TOL)] + flags) == 2


@pytest.mark.parametrize("count,support", [(3, 256), (4, 100)])
def test_refresh_many_pairs_complex_slots(count, support):
    """refresh_many under S2C-first packs the real values in pairs, one
    complex-slot bootstrap each (the odd one alone), and unpacks them:
    every value within the two-pass tolerance of one refresh each, masked
    to the support."""
    slots = 1 << 11
    cc, keys = P.build_context(slots, ring_dim=1 << 12, seed=5)
    ev = P.PackedEvaluator(cc, keys, slots, s2c_first=True, level_budget=(3, 3))
    rng = np.random.default_rng(count)
    xs = [rng.uniform(-3, 3, slots) for _ in range(count)]
    cts = [ev.encrypt(x) for x in xs]
    b0 = ev.stats["bootstraps"]
    outs = ev.refresh_many(cts, 4.0, support, passes=2)
    assert ev.stats["bootstraps"] - b0 == 2 * ((count + 1) // 2)
    singles = [ev.refresh(ct, 4.0, support, passes=2) for ct in cts]
    for x, o, s in zip(xs, outs, singles):
        want = np.where(np.arange(slots) < support, x, 0.0)
        got, one = ev.decrypt(o, slots), ev.decrypt(s, slots)
        assert np.max(np.abs(got - want)) < TOL
        assert np.max(np.abs(one - want)) < TOL
        assert o.GetLevel() == s.GetLevel()
