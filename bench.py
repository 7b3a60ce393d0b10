#!/usr/bin/env python3
"""Benchmark of the CKKS evaluation hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one step): the hoisted rotation set {+-2^k : k = 0..14} (30
rotations: one shared ModUp, then per rotation the key inner product,
ModDown and the Galois permutation) applied to one ciphertext at N = 2^16,
L = 24 limbs, K = 8 special primes, dnum = 3, plus one rescale.  Inputs
are seeded synthetic ciphertext residues and seeded Galois keys, all
resident in HBM before the timed region.  `value` is rotations/s.

The same run also times the raw NTT / MAC batch (64 ciphertexts x 2 polys
x 24 limbs at N = 2^16: forward NTT, plaintext MAC over the 64
ciphertexts, inverse NTT) and reports NTT HBM GB/s, one encrypted Mamba-2
SSM layer step at the 130M shape, and EvalBootstrap at N = 2^16 (one pass
and the two-pass refresh, 45 limbs), and a 24-layer encrypted Mamba-2 decode
(s/token, first and carried-state token) at N = 2^16 and at the audited
classical-128 setting (N = 2^17).

Per-kernel times come from HIP events recorded on the library's stream
around every launch (fhe_profile_begin / fhe_profile_end) over a profiled
repeat of the timed steps.  The CPU baseline times this build's C
restatement of the same algorithms (the oracle; OpenFHE is not on this
host) on a bounded sample, single-threaded for rotations and on all
available cores for the NTT.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "fhe-mamba_amd"))

METRIC = "rotations/s (N=2^16,L=24,hybrid KS); NTT HBM GB/s; s/token M2-130M"
HBM_PEAK = 8.0e12  # B/s, MI355X HBM3E
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE on this workload (FETCH_SIZE x 2.0, WRITE_SIZE x 1.0, the factors
# a plain copy of known size reads back); recorded in
# profiles/rotation_step_n65536_l24.md together with the commands and the
# hash of the kernel sources they were measured on.  A build from other
# sources reports traffic as null.
MEASURED_TRAFFIC = {
    "csrc_sha16": "d4c33860f0b17125",
    "kernels": {
        # 30-rotation batch launches of the rotation step
        "ntt_fwd_blocks_moddown": 3_096_629_069 + 754_974_720,
        "k_moddown_mid": 253_267_354 + 758_981_414,
        "ntt_inv_blocks_ksk": 776_270_925 + 251_658_240,
        # NTT batch (64 ciphertexts x 2 polys x 24 limbs): one pass, and the MAC
        "ntt_pass": 1_636_261_914 + 1_610_612_736,
        "k_mac": 2_416_047_309 + 25_165_824,
    },
}


def csrc_sha16() -> str:
    """First 16 hex digits of the SHA-256 over the library's kernel sources
    (fhe-mamba_amd/csrc, file names and contents in name order)."""
    import hashlib
    d = os.path.join(ROOT, "fhe-mamba_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(d)):
        h.update(name.encode())
        with open(os.path.join(d, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic(kernel: str):
    if MEASURED_TRAFFIC["csrc_sha16"] != csrc_sha16():
        return None
    return MEASURED_TRAFFIC["kernels"].get(kernel)
LOG_N, DEPTH, SCALE_BITS, FIRST_BITS, DNUM = 16, 23, 59, 60, 3
N = 1 << LOG_N
LIMB = N * 8  # bytes per limb
STEPS = [s * (1 << k) for k in range(15) for s in (1, -1)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def rotation_bytes(L: int, K: int) -> tuple[int, int, int]:
    """Algorithmic HBM bytes of one step: ciphertext read once, per hoisted
    rotation the key ([dnum][2][L+K] limbs) read and the output written,
    plus the rescale (read 2 x L limbs, write 2 x (L-1))."""
    ct = 2 * L * LIMB
    per_rot = DNUM * 2 * (L + K) * LIMB + ct
    rescale = 2 * L * LIMB + 2 * (L - 1) * LIMB
    return ct, per_rot, rescale


def run_rotations(F, steps: int, warmup: int):
    import numpy as np

    q, p = F.gen_moduli(LOG_N, DEPTH, SCALE_BITS, FIRST_BITS, DNUM)
    ctx = F.Context(LOG_N, q, p, DNUM)
    L, K = ctx.L, ctx.K
    log(f"rotation context: N=2^{LOG_N} L={L} K={K} dnum={ctx.dnum} alpha={ctx.alpha}")
    s = ctx.keygen_secret(1)
    gal = [F.galois_element(r, N) for r in STEPS]
    keys = [ctx.keygen_galois(s, g, 1000 + i) for i, g in enumerate(gal)]
    rng = np.random.default_rng(7)
    ct_host = np.empty((2, L, N), dtype=np.uint64)
    for j, qj in enumerate(q):
        ct_host[:, j, :] = rng.integers(0, qj, (2, N), dtype=np.uint64)
    ct = ctx.upload(ct_host)
    outs = [ctx.poly(2, L) for _ in STEPS]
    rs_out = ctx.poly(2, L - 1)

    def step():
        digits = ctx.rotation_precompute(ct)
        ctx.rotate_hoisted(ct, digits, keys, gal, outs)
        ctx.rescale(ct, out=rs_out)
        digits.close()

    for _ in range(warmup):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    ctx.profile_begin()
    for _ in range(steps):
        step()
    prof = ctx.profile_end()
    # Non-hoisted rotations (each with its own ModUp), same keys and input.
    single = ctx.poly(2, L)
    for k, g in zip(keys[:4], gal[:4]):
        ctx.rotate(ct, k, g, out=single)
    ctx.sync()
    t1 = time.perf_counter()
    for k, g in zip(keys, gal):
        ctx.rotate(ct, k, g, out=single)
    ctx.sync()
    single_s = time.perf_counter() - t1
    ct_b, rot_b, rs_b = rotation_bytes(L, K)
    step_bytes = ct_b + len(STEPS) * rot_b + rs_b
    res = {
        "elapsed_s": elapsed,
        "ms_per_step": 1e3 * elapsed / steps,
        "rotations_per_s": len(STEPS) * steps / elapsed,
        "single_rotations_per_s": len(keys) / single_s,
        "step_bytes": step_bytes,
        "profile": prof,
        "L": L,
        "K": K,
    }
    for k in keys:
        k.close()
    ctx.close()
    return res


def run_ntt_batch(F, steps: int, warmup: int, count: int = 64):
    import numpy as np

    q = [int(x) for x in ntt_primes(LOG_N, 60, 24)]
    ctx = F.Context(LOG_N, q, [], 1)
    L = len(q)
    rng = np.random.default_rng(11)
    x = ctx.poly(2 * count, L)
    w = ctx.poly(count, L)
    host = np.empty((2 * count, L, N), dtype=np.uint64)
    for j, qj in enumerate(q):
        host[:, j, :] = rng.integers(0, qj, (2 * count, N), dtype=np.uint64)
    x = ctx.upload(host)
    w = ctx.upload(host[:count].copy())
    del host
    acc = ctx.poly(2, L)

    def step():
        ctx.ntt_forward_dev(x.data_ptr(), 2 * count, L, 0)
        ctx.mac_dev(x.data_ptr(), w.data_ptr(), count, L, acc.data_ptr())
        ctx.ntt_inverse_dev(x.data_ptr(), 2 * count, L, 0)

    for _ in range(warmup):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    ctx.profile_begin()
    for _ in range(steps):
        step()
    prof = ctx.profile_end()
    ntt_bytes = 2 * count * L * LIMB * 2  # read + write the batch once
    mac_bytes = (2 * count * L + count * L + 2 * L) * LIMB
    t_fwd = sum(prof.get(k, (0, 0.0))[1] for k in ("ntt_fwd_cols", "ntt_fwd_blocks")) / steps
    t_inv = sum(prof.get(k, (0, 0.0))[1] for k in ("ntt_inv_cols", "ntt_inv_blocks")) / steps
    t_mac = prof.get("k_mac", (0, 0.0))[1] / steps
    ctx.close()
    return {
        "elapsed_s": elapsed,
        "ms_per_step": 1e3 * elapsed / steps,
        "ntt_gbps": 2 * ntt_bytes / ((t_fwd + t_inv) * 1e-3) / 1e9,
        "ntt_fwd_ms": t_fwd,
        "ntt_inv_ms": t_inv,
        "mac_ms": t_mac,
        "mac_gbps": mac_bytes / (t_mac * 1e-3) / 1e9 if t_mac else None,
        "ntt_bytes": ntt_bytes,
        "profile": prof,
    }


def run_ssm_step(steps: int = 2, warmup: int = 1):
    """One encrypted Mamba-2 SSM layer step at the 130M shape (24 heads x 64
    channels x 128 states in six 32768-slot state ciphertexts) at N=2^16,
    24 limbs: decay exp(dt A), state update, rotate-sum readout, D x.  Inputs
    are seeded synthetic values with the model's distributions, encrypted
    before timing; the result is decrypted after timing and compared with
    the float64 reference."""
    import numpy as np
    from fhemamba_amd.ckks_probes import build_toy_context
    from fhemamba_amd.mamba2 import (DecayPolynomial, EncryptedSSMStep, SSMShape,
                                     expand_channels, expand_heads, expand_states, pack_state,
                                     ssm_step_reference, unpack_state)

    s = SSMShape()
    rng = np.random.default_rng(5)
    h = rng.normal(0, 0.5, (s.nheads, s.headdim, s.d_state))
    x = np.clip(rng.normal(0, 1, (s.nheads, s.headdim)), -8, 8)
    dt = np.clip(np.log1p(np.exp(rng.normal(0, 1, s.nheads))), 0.0, 6.0)
    A = -np.exp(rng.uniform(0, np.log(16), s.nheads))
    B, C = rng.normal(0, 0.3, s.d_state), rng.normal(0, 0.3, s.d_state)
    D = rng.normal(0, 1, s.nheads)
    cc, keys = build_toy_context(ring_dimension=N, batch=s.slots, depth=DEPTH,
                                 scale_bits=SCALE_BITS, first_mod_bits=FIRST_BITS, seed=11)
    step = EncryptedSSMStep(cc, keys, s, A, D, DecayPolynomial(amax=96.0, squarings=5,
                                                               degree=13))
    cc.EvalRotateKeyGen(keys.secretKey, step.rotation_indices())

    def enc(v):
        return cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(v)))

    xc = np.zeros(s.slots)
    xc[: s.d_inner] = x.reshape(-1)
    inputs = ([enc(v) for v in pack_state(h, s)], [enc(v) for v in expand_channels(x, s)],
              [enc(v) for v in expand_heads(dt, s)], enc(expand_states(B, s)),
              enc(expand_states(C, s)), enc(xc))
    for _ in range(warmup):
        step(*inputs)
    cc.device.sync()
    t0 = time.perf_counter()
    for _ in range(steps):
        new_state, y = step(*inputs)
    cc.device.sync()
    per_step = (time.perf_counter() - t0) / steps

    def dec(ct):
        pt = cc.Decrypt(ct, keys.secretKey)
        pt.SetLength(s.slots)
        return np.asarray(pt.GetRealPackedValue())

    h2, y_ref = ssm_step_reference(h, x, dt, A, B, C, D)
    err_h = float(np.max(np.abs(unpack_state([dec(c) for c in new_state], s) - h2)))
    err_y = float(np.max(np.abs(dec(y)[: s.d_inner].reshape(s.nheads, s.headdim) - y_ref)))
    return {
        "s_per_layer_step": per_step,
        "max_abs_err_state": err_h,
        "max_abs_err_y": err_y,
        "levels_used": int(y.GetLevel()),
        "workload": ("Mamba-2-130M SSM layer step (24 heads x 64 x 128 states, six 32768-slot "
                     "state ciphertexts), N=2^16, 24 limbs, synthetic seeded inputs"),
    }


BOOT_DEPTH, BOOT_BUDGET = 44, (4, 4)
# 1,083.2 s of bootstrapping over 2,187 EvalBootstrap calls in the reference's
# Mamba-2-130M decode on GB10 (results/dgx/2026-09-24/owned-arithmetic/
# m2-full-candidate/native.json, `timing` and `operation_counts`).
REF_BOOTSTRAP_S = 1083.2 / 2187


def _bootstrap_once(secret_dist: str, steps: int, warmup: int, s2c_first: bool = False) -> dict:
    import numpy as np
    from fhemamba_amd.ckks_probes import build_toy_context

    slots = N // 2
    cc, keys = build_toy_context(ring_dimension=N, batch=slots, depth=BOOT_DEPTH,
                                 scale_bits=SCALE_BITS, first_mod_bits=FIRST_BITS, seed=21,
                                 secret_dist=secret_dist)
    cc.EvalBootstrapSetup(list(BOOT_BUDGET), [0, 0], slots, s2c_first=s2c_first,
                          real_slots=s2c_first)
    cc.EvalBootstrapKeyGen(keys.secretKey, slots)
    x = np.random.default_rng(8).uniform(-1, 1, slots)
    ct = cc.Encrypt(keys.publicKey, cc.MakeCKKSPackedPlaintext(list(x)))
    ct.SetLevel(cc.GetBootstrapInputCeiling())
    res = {}
    for passes in (1, 2):
        for _ in range(warmup):
            cc.EvalBootstrap(ct, passes)
        cc.device.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            out = cc.EvalBootstrap(ct, passes)
        cc.device.sync()
        sec = (time.perf_counter() - t0) / steps
        pt = cc.Decrypt(out, keys.secretKey)
        pt.SetLength(slots)
        err = float(np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - x)))
        res[f"{'one' if passes == 1 else 'two'}_pass"] = {
            "ms": sec * 1e3, "max_abs_err": err, "log2_err": float(np.log2(err))}
    if not s2c_first:
        # the client's public coefficient bound of its slots (the ordinary
        # order's EvalMod sees the coefficients): less scale-down
        from fhemamba_amd.bootstrap import coefficient_bound
        b = coefficient_bound(x)
        out = cc.EvalBootstrap(ct, 1, coeff_bound=b)
        pt = cc.Decrypt(out, keys.secretKey)
        pt.SetLength(slots)
        err = float(np.max(np.abs(np.asarray(pt.GetRealPackedValue()) - x)))
        res["one_pass_coeff_bound"] = {"coeff_bound": b, "max_abs_err": err,
                                       "log2_err": float(np.log2(err))}
    sine = cc._boot.cfg.sine
    res.update({
        "levels_consumed": cc.GetBootstrapDepth(),
        "input_ceiling": cc.GetBootstrapInputCeiling(),
        "output_level": int(out.GetLevel()),
        "rotation_keys": len(cc._boot.rotation_indices()),
        "eval_mod": {"K": sine.K, "double_angles": sine.r, "degree": sine.degree},
    })
    return res


def run_bootstrap(steps: int = 3, warmup: int = 2):
    """EvalBootstrap of one full-packing ciphertext (32768 slots) at N=2^16,
    45 limbs (multiplicative depth 44, 59-bit scale, 60-bit q0), dnum 3,
    level budget (4, 4): one pass and the two-pass refresh, for a
    uniform-ternary secret (K = 512) and a sparse-ternary one (h = 192,
    K = 64; the reference decoder's default).  The input is a seeded
    uniform vector in [-1, 1], encrypted and brought to the last level but
    one before timing; errors are measured after timing."""
    import gc
    res = _bootstrap_once("UNIFORM_TERNARY", steps, warmup)
    gc.collect()  # each context holds its own bootstrapping keys
    res["sparse_secret"] = _bootstrap_once("SPARSE_TERNARY", steps, warmup)
    gc.collect()
    res["s2c_first"] = _bootstrap_once("UNIFORM_TERNARY", steps, warmup, True)
    gc.collect()
    res["s2c_first_sparse_secret"] = _bootstrap_once("SPARSE_TERNARY", steps, warmup, True)
    res.update({
        "reference_gb10_ms_per_bootstrap": REF_BOOTSTRAP_S * 1e3,
        "speedup_vs_reference_one_pass": REF_BOOTSTRAP_S / (res["one_pass"]["ms"] * 1e-3),
        "speedup_vs_reference_one_pass_sparse":
            REF_BOOTSTRAP_S / (res["sparse_secret"]["one_pass"]["ms"] * 1e-3),
        "workload": ("EvalBootstrap, 32768 slots, N=2^16, 45 limbs (depth 44, scale 2^59), "
                     "dnum 3, level budget (4,4); uniform ternary secret (K=512) at the top "
                     "level, sparse ternary (h=192, K=64) under sparse_secret; the reference "
                     "figure is its GB10 mean over a full decode (sparse secret)"),
    })
    return res


# 396.6 s per carried-state token (mean of 4) and 356.4 s for the first, the
# reference's Mamba-2-130M encrypted decode on GB10 (results/dgx/2026-09-24/
# owned-arithmetic/m2-full-candidate/native.json, `timing`).
REF_TOKEN_S = 396.6


# carried tokens decoded to cover one refresh cycle of the carried SSM
# state in the N=2^16 decode: its level grows by one a token until its six
# groups are refreshed together, every eighth carried token on this payload
STATE_CYCLE = 8


def run_decode(tokens: int = 1 + STATE_CYCLE, security: str = "not-set"):
    """Encrypted Mamba-2 decode of a seeded random-init 24-layer payload at
    the 130M shape (d_model 768, d_inner 1536, 24 heads x 64, state 128,
    conv 4), depth 44, 59-bit scale; the first token from zero state, then
    carried-state tokens: the carried figure is the mean of the first four
    (the reference's protocol: five tokens, the mean of the four carried
    ones), the cycle figure the mean over one full refresh cycle of the
    carried state (STATE_CYCLE tokens, the state-refresh token included).
    Errors against the payload's polynomial circuit after decryption.
    security "not-set": N=2^16, 32768 slots, sparse ternary secret (the
    reference decoder's); "128-classic": the audited classical-128 setting,
    N=2^17, 65536 slots, 45 Q + 12 P primes, four digits, uniform ternary
    secret."""
    import tempfile
    from fhemamba_amd import mamba2_decode as D
    from fhemamba_amd import mamba2_payload as M
    with tempfile.TemporaryDirectory() as d:
        M.synthetic_chain(d, n_layers=24, n_test_tokens=tokens, seed=13)
        rep = D.run_payload(d, seed=14, security=security, log=lambda m: None)
    per, passes = rep["seconds_per_token"], rep["per_token_bootstraps"]
    carried = sum(per[1:5]) / len(per[1:5]) if len(per) > 1 else None
    # the cycle ends at the carried token that refreshes the state groups
    # (the most bootstrap passes, more than the first carried token's)
    end = max(range(1, len(per)), key=lambda k: passes[k], default=None)
    cycle = (sum(per[1:end + 1]) / end
             if end is not None and passes[end] > passes[1] else None)
    if security == "128-classic":
        a = rep["security_audit"]
        return {
            "s_per_token_first": rep["first_token_seconds"],
            "s_per_token_carried": carried,
            "s_per_token_all": rep["seconds_per_token"],
            "max_abs_err_vs_polynomial": rep["max_abs_error_vs_polynomial"],
            "bootstraps_per_token": rep["bootstraps"] / tokens,
            "rotations_per_token": rep["rotations"] / tokens,
            "security_audit": {k: a[k] for k in ("ring_dimension", "q_bits", "p_bits",
                                                 "qp_bits", "q_towers", "p_towers",
                                                 "hybrid_digits", "guideline_max_qp_bits",
                                                 "passed")},
            "secret_key_dist": rep["secret_key_dist"],
            "workload": ("encrypted Mamba-2-130M-shaped decode, 24 layers (seeded random-init "
                         "weights, synthetic payload), classical-128: N=2^17, 65536 slots, "
                         "depth 44, 45 Q + 12 P primes, 4 digits, uniform ternary secret, "
                         "SlotToCoeff-first two-pass refreshes (one pass before a Newton "
                         "step); first token from zero state, then carried state"),
        }
    return {
        "s_per_token_first": rep["first_token_seconds"],
        "s_per_token_carried": carried,
        "s_per_token_cycle": cycle,
        "state_refresh_token": (end + 1) if cycle is not None else None,
        "s_per_token_all": rep["seconds_per_token"],
        "bootstrap_passes_per_token": rep["per_token_bootstraps"],
        "max_abs_err_vs_polynomial": rep["max_abs_error_vs_polynomial"],
        "bootstraps_per_token": rep["bootstraps"] / tokens,
        "rotations_per_token": rep["rotations"] / tokens,
        "reference_gb10_s_per_token": REF_TOKEN_S,
        "speedup_vs_reference": REF_TOKEN_S / carried if carried else None,
        "secret_key_dist": rep["secret_key_dist"],
        "workload": ("encrypted Mamba-2-130M-shaped decode, 24 layers (seeded random-init "
                     "weights and calibrated polynomials, synthetic payload), N=2^16, "
                     "depth 44, sparse-ternary secret (h=192) as the reference decoder's, "
                     "SlotToCoeff-first refreshes (two passes at the precision-critical "
                     "sites); first token from zero state, then carried state; carried: "
                     "mean of tokens 2-5; cycle: mean of the carried tokens up to the one "
                     "that refreshes the state's six groups (state_refresh_token, 1-based), "
                     "one refresh cycle of the carried state"),
    }


def ntt_primes(log_n: int, bits: int, count: int):
    """Descending primes q = 1 mod 2N below 2^bits (deterministic)."""
    from fhemamba_amd.core import gen_moduli  # noqa: F401  (library must load)

    m = 2 << log_n
    out, c = [], ((1 << bits) // m) * m + 1
    while len(out) < count:
        c -= m
        if _is_prime(c):
            out.append(c)
    return out


def _is_prime(n: int) -> bool:
    if n < 2:
        return False
    for b in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37):
        if n % b == 0:
            return n == b
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for b in (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37):
        x = pow(b, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def _cpu_threads() -> tuple[int, int]:
    """(threads used for the all-core figures, nproc): the cores this process
    may run on, capped by OMP_NUM_THREADS when set and by 16 (a one-GPU
    share of the host)."""
    nproc = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    omp = int(os.environ.get("OMP_NUM_THREADS") or usable)
    return max(1, min(usable, omp, 16)), nproc


class OpTally:
    """Counts the library calls a decode makes, by operation class and limb
    count, by wrapping the device-context methods (fhemamba_amd.core.Context)
    for the duration of a `with` block.  Classes:
      ks      full key switch with its own ModUp (rotate, keyswitch,
              relinearize, each ciphertext of rotate_many and each tensor of
              relinearize_many, each Horner or batched giant step of a
              linear transform);
      modup   a shared ModUp (rotation_precompute; the babies of a linear
              transform);
      hks     a hoisted key switch from shared digits (each key of
              rotate_hoisted; each rotated baby of a linear transform);
      rescale (each input of rescale_many too), tensor, modraise;
      pmul    one plaintext or constant product over 2 polys (mul_plain,
              mul_const, mul_int, each diagonal of a linear transform, each
              term of linear_wsum);
      add     one elementwise addition-class op over 2 polys;
      encode  one encoded vector (per row of encode_many).
    `snapshot()` returns the counts so far; the decode's per-token counts are
    differences of snapshots taken before each step."""

    def __init__(self, Context):
        import collections
        self.Context = Context
        self.counts = collections.Counter()
        self._saved = {}

    def _wrap(self, name, tally):
        orig = getattr(self.Context, name)
        self._saved[name] = orig

        def wrapper(ctx, *a, **k):
            tally(*a, **k)
            return orig(ctx, *a, **k)
        setattr(self.Context, name, wrapper)

    def __enter__(self):
        c = self.counts

        def one(cls, pos=0):
            return lambda *a, **k: c.update({(cls, a[pos].nlimb): 1})

        def lt(ct, pts, bstep, baby_keys, *rest, giant_keys=None, hoisted=False, **k):
            n = ct.nlimb
            count = len(pts)
            giants = -(-count // bstep)
            c[("pmul", n)] += sum(p is not None for p in pts)
            c[("modup", n)] += 1
            c[("hks", n)] += sum(x is not None for x in baby_keys)
            c[("ks", n)] += max(0, giants - 1)

        for name in ("add", "sub", "negate", "add_plain", "add_const"):
            self._wrap(name, one("add"))
        for name in ("mul_plain", "mul_const", "mul_int"):
            self._wrap(name, one("pmul"))
        for name in ("keyswitch", "relinearize", "rotate"):
            self._wrap(name, one("ks"))
        self._wrap("rescale", one("rescale"))
        self._wrap("tensor", one("tensor"))
        self._wrap("rotation_precompute", one("modup"))
        self._wrap("mod_raise", lambda a, nlimb, *r, **k: c.update({("modraise", nlimb): 1}))
        self._wrap("linear_wsum",
                   lambda terms, w, nlimb, *r, **k: c.update({("pmul", nlimb): len(terms)}))
        self._wrap("rotate_hoisted",
                   lambda ct, d, keys, *r, **k: c.update({("hks", ct.nlimb): len(keys)}))
        self._wrap("rotate_many",
                   lambda cts, *r, **k: c.update([("ks", x.nlimb) for x in cts]))
        self._wrap("relinearize_many",
                   lambda ts, *r, **k: c.update([("ks", x.nlimb) for x in ts]))
        self._wrap("rescale_many",
                   lambda ps, *r, **k: c.update([("rescale", x.nlimb) for x in ps]))
        self._wrap("linear_transform", lambda *a, **k: lt(*a, **k))
        self._wrap("linear_transform_hoisted", lambda *a, **k: lt(*a, **k))
        self._wrap("encode", lambda v, slots, scale, nlimb, *r, **k:
                   c.update({("encode", nlimb): 1}))
        self._wrap("encode_many", lambda rows, slots, scale, nlimb, *r, **k:
                   c.update({("encode", nlimb): len(rows)}))
        return self

    def __exit__(self, *exc):
        for name, orig in self._saved.items():
            setattr(self.Context, name, orig)
        self._saved.clear()

    def snapshot(self):
        return dict(self.counts)


def count_decode_ops(tokens: int = 2):
    """Library operations of one carried-state token of the 24-layer decode
    at N = 2^16 (the decode workload's payload and parameters): a separate
    pass with the tally installed, so the timed decode runs unwrapped."""
    import tempfile
    from fhemamba_amd import core
    from fhemamba_amd import mamba2_decode as D
    from fhemamba_amd import mamba2_payload as M
    snaps = []
    step = D.EncryptedMamba2Decoder.step
    with tempfile.TemporaryDirectory() as d, OpTally(core.Context) as tally:
        M.synthetic_chain(d, n_layers=24, n_test_tokens=tokens, seed=13)

        def counted(dec, *a, **k):
            snaps.append(tally.snapshot())
            return step(dec, *a, **k)
        D.EncryptedMamba2Decoder.step = counted
        try:
            D.run_payload(d, seed=14, log=lambda m: None)
        finally:
            D.EncryptedMamba2Decoder.step = step
        snaps.append(tally.snapshot())
    last, prev = snaps[-1], snaps[-2]
    return {k: v - prev.get(k, 0) for k, v in last.items() if v - prev.get(k, 0)}


def cpu_decode_estimate(ops: dict, threads: int, parallel_speedup: float) -> dict:
    """Seconds per carried-state token of the 24-layer decode on the host
    CPU, estimated: the token's library operations (count_decode_ops) times
    the oracle's measured time for each operation class at N = 2^16 on one
    thread, interpolated linearly in the limb count between the measured
    levels.  The all-threads figure divides by the oracle's measured
    limb-parallel speed-up (its batched NTT on `threads` threads), the way a
    CPU library parallelises these operations over limbs.  An estimate of a
    port of these algorithms, not a run of OpenFHE."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    q, p = O.gen_moduli(LOG_N, 44, SCALE_BITS, FIRST_BITS, DNUM)
    c = O.Ctx(LOG_N, q, p, DNUM)
    s = c.secret(1)
    g = O.galois_elt(1, N)
    key = c.galois_key(s, g, 5)
    rng = np.random.default_rng(9)
    levels = [4, 12, 24, 34, 45]
    ct_full = np.stack([np.stack([rng.integers(0, qj, N, dtype=np.uint64) for qj in q])
                        for _ in range(2)])
    vals = rng.uniform(-1, 1, N // 2)

    def t(fn, reps=1):
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) / reps

    table = {k: [] for k in ("ks", "modup", "hks", "rescale", "tensor", "pmul", "add",
                             "modraise", "encode")}
    for nq in levels:
        ct = np.ascontiguousarray(ct_full[:, :nq])
        dig = c.modup(ct[1])
        table["ks"].append(t(lambda: c.rotate(ct, key, g)))
        table["modup"].append(t(lambda: c.modup(ct[1])))
        table["hks"].append(t(lambda: c.rotate_hoisted(ct, dig, key, g)))
        table["rescale"].append(t(lambda: c.rescale(ct)))
        table["tensor"].append(t(lambda: c.tensor(ct, ct), 2))
        table["pmul"].append(t(lambda: c.mac(ct[None], ct[:1, :, :]), 3))
        table["add"].append(t(lambda: c.add(ct, ct), 3))
        table["modraise"].append(t(lambda: (c.ntt_inv_batch(ct[:, :1]),
                                            c.ntt_fwd_batch(ct, 0))))
        table["encode"].append(t(lambda: c.encode(vals, N // 2, 2.0**59, nq)))

    def cost(cls, nq):
        return float(np.interp(nq, levels, table[cls]))

    total, by_class = 0.0, {}
    for (cls, nq), n in ops.items():
        sec = n * cost(cls, nq)
        by_class[cls] = by_class.get(cls, 0.0) + sec
        total += sec
    return {
        "one_thread": total,
        "all_threads": total / parallel_speedup,
        "threads": threads,
        "parallel_speedup": parallel_speedup,
        "seconds_by_class_one_thread": by_class,
        "operations_per_token": {cls: sum(n for (k, _), n in ops.items() if k == cls)
                                 for cls in table},
        "oracle_seconds_one_thread": {"levels": levels, **table},
    }


def cpu_baseline(budget_s: float = 24.0, decode_ops: dict | None = None):
    """The oracle (this build's scalar C restatement of the same algorithms;
    OpenFHE is not installed on this host) at the benchmark shape on a
    bounded sample:
      * hoisted rotations from one shared ModUp (the GPU step's operation),
        on one thread and on all threads (independent rotations of the set
        in parallel, the ModUp once), with the GPU step's ModUp and rescale
        amortised over 30 rotations for the headline figure;
      * non-hoisted rotations (own ModUp each) on one thread;
      * the forward NTT of 8 ciphertexts x 24 limbs on one and all threads."""
    import concurrent.futures as cf

    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    threads, nproc = _cpu_threads()
    q, p = O.gen_moduli(LOG_N, DEPTH, SCALE_BITS, FIRST_BITS, DNUM)
    c = O.Ctx(LOG_N, q, p, DNUM)
    s = c.secret(1)
    rng = np.random.default_rng(7)
    ct = np.stack([np.stack([rng.integers(0, qj, N, dtype=np.uint64) for qj in q])
                   for _ in range(2)])
    steps = (1, -1, 2, -2)
    keys = [(O.galois_elt(r, N), c.galois_key(s, O.galois_elt(r, N), 1000 + i))
            for i, r in enumerate(steps)]

    def timed(fn, min_s, min_n=1):
        n, t0 = 0, time.perf_counter()
        while n < min_n or time.perf_counter() - t0 < min_s:
            fn(n)
            n += 1
        return n, time.perf_counter() - t0

    t0 = time.perf_counter()
    digits = c.modup(ct[1])
    modup_s = time.perf_counter() - t0
    t0 = time.perf_counter()
    c.rescale(ct)
    rescale_s = time.perf_counter() - t0

    def hoisted(i):
        g, k = keys[i % len(keys)]
        c.rotate_hoisted(ct, digits, k, g)

    n1, t1 = timed(hoisted, budget_s * 0.15, 2)
    one_core = n1 / t1
    with cf.ThreadPoolExecutor(threads) as ex:
        jobs = 2 * threads
        t0 = time.perf_counter()
        list(ex.map(hoisted, range(jobs)))
        all_core = jobs / (time.perf_counter() - t0)

    def single(i):
        g, k = keys[i % len(keys)]
        c.rotate(ct, k, g)

    n2, t2 = timed(single, budget_s * 0.15, 2)
    rots = len(STEPS)
    step_all = modup_s + rots / all_core + rescale_s
    step_one = modup_s + rots / one_core + rescale_s

    qn = [int(x) for x in ntt_primes(LOG_N, 60, 24)]
    cn = O.Ctx(LOG_N, qn, [], 1)
    batch = np.stack([np.stack([rng.integers(0, qj, N, dtype=np.uint64) for qj in qn])
                      for _ in range(8)])
    ntt_bytes = batch.size * 8 * 2  # read + write once

    def ntt_rate(nthreads):
        n, t = timed(lambda i: cn.ntt_fwd_batch(batch, 0, nthreads=nthreads),
                     budget_s * 0.1, 1)
        return n * ntt_bytes / t / 1e9

    ntt_one, ntt_all = ntt_rate(1), ntt_rate(threads)
    decode = None
    if decode_ops:
        decode = cpu_decode_estimate(decode_ops, threads, ntt_all / ntt_one)
        decode = {"kind": "port-estimate",
                  "s_per_token_one_thread": decode["one_thread"],
                  "s_per_token_all_threads": decode["all_threads"],
                  "workload": ("one carried-state token of the 24-layer Mamba-2-130M-shaped "
                               "decode at N=2^16, depth 44 (the mamba2_decode workload): its "
                               "library operations counted by class and limb count, times the "
                               "oracle's measured one-thread time of each class at N=2^16 "
                               "(interpolated in the limb count); all threads: divided by the "
                               "oracle's measured limb-parallel speed-up"),
                  **{k: v for k, v in decode.items() if k not in ("one_thread", "all_threads")}}
    return {
        "value": rots / step_all,
        "unit": "rotations/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"hoisted-set rotations of one N=2^16, L=24, K=8, dnum=3 ciphertext by the "
                   f"scalar C oracle: {jobs} rotations on {threads} threads (steps +-1, +-2), "
                   f"one ModUp and one rescale amortised over {rots} rotations as in the GPU "
                   f"step; OpenFHE CPU: unavailable on this host"),
        "nproc": nproc,
        "hoisted_rotations_per_s_all_threads_amortised": rots / step_all,
        "hoisted_rotations_per_s_one_thread_amortised": rots / step_one,
        "hoisted_rotation_only_per_s": {"one_thread": one_core, "all_threads": all_core},
        "single_rotations_per_s_one_thread": n2 / t2,
        "modup_s": modup_s,
        "rescale_s": rescale_s,
        "ntt_gbps": {"one_thread": ntt_one, "all_threads": ntt_all},
        "ntt_sample": "forward NTT of 8 ciphertexts x 24 limbs (60-bit primes) at N=2^16",
        "decode_s_per_token": decode,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-ntt", action="store_true")
    ap.add_argument("--skip-ssm", action="store_true")
    ap.add_argument("--skip-bootstrap", action="store_true")
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the workloads, run one plain limb copy (k_copy_limbs) of "
                         f"{COPY_PROBE_BYTES} bytes read and the same written, untimed, as "
                         "the reference point for hardware byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}): the path has no "
              "multi-GPU component in this build (one GPU's share of a sharded run is what it "
              "measures).",
              file=sys.stderr)
        return 2
    import fhemamba_amd as F

    log("rotation workload")
    rot = run_rotations(F, args.steps, args.warmup)
    ntt = None if args.skip_ntt else (log("ntt batch workload"),
                                      run_ntt_batch(F, args.steps, args.warmup))[1]
    prof = rot["profile"]
    model = step_kernel_bytes(rot["L"], rot["K"], len(STEPS))
    dom = max(prof, key=lambda k: prof[k][1])
    launches, total_ms = prof[dom]
    avg_s = total_ms * 1e-3 / launches
    per_launch = model[dom] * args.steps / launches if dom in model else None
    achieved = per_launch / avg_s if per_launch else None
    roofline = {
        "bound": "hbm",
        "kernel": dom,
        "achieved": achieved / 1e9 if achieved else None,
        "peak": HBM_PEAK / 1e9,
        "unit": "GB/s",
        "frac": achieved / HBM_PEAK if achieved else None,
        "traffic": measured_traffic(dom),
        "csrc_sha16": csrc_sha16(),
        "bytes_per_launch": per_launch,
        "avg_launch_us": avg_s * 1e6,
        "step_frac": rot["step_bytes"] / (rot["ms_per_step"] * 1e-3) / HBM_PEAK,
    }
    kernel_gbps = {k: model[k] * args.steps / (prof[k][1] * 1e-3) / 1e9
                   for k in sorted(prof) if k in model and prof[k][1] > 0}
    out = {
        "metric": METRIC,
        "value": rot["rotations_per_s"],
        "unit": "rotations/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": rot["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic (seeded residues, seeded Galois keys)",
        "config": {
            "workload": "hoisted rotation set {+-2^k, k<15} (30 rotations) + rescale on one "
                        "ciphertext, N=2^16, L=24, K=8, dnum=3",
            "ring_dim": N, "limbs": rot["L"], "special_primes": rot["K"], "dnum": DNUM,
            "rotations_per_step": len(STEPS), "parallelism": "single GPU",
        },
        "roofline": roofline,
        "kernels_ms_per_step": {k: v[1] / args.steps for k, v in sorted(prof.items())},
        "kernels_gbps": kernel_gbps,
        "single_rotation": {
            "rotations_per_s": rot["single_rotations_per_s"],
            "workload": "the same 30 rotations, each a full EvalRotate (own ModUp)",
            "frac": rot["single_rotations_per_s"] * 150_994_944 / HBM_PEAK,
        },
    }
    if ntt:
        out["ntt"] = {k: ntt[k] for k in ("ntt_gbps", "ntt_fwd_ms", "ntt_inv_ms", "mac_ms",
                                          "mac_gbps", "ms_per_step")}
        out["ntt"]["workload"] = ("64 ciphertexts x 2 polys x 24 limbs, N=2^16: forward NTT, "
                                  "MAC over 64 plaintexts, inverse NTT")
        out["ntt"]["frac"] = ntt["ntt_gbps"] * 1e9 / HBM_PEAK
        # counter-measured HBM bytes of one two-pass NTT launch over the
        # batch (each pass reads and writes every limb) and of the MAC
        out["ntt"]["traffic_per_pass"] = measured_traffic("ntt_pass")
        out["ntt"]["mac_traffic"] = measured_traffic("k_mac")
    # Each leg builds its own context and keys (tens of GB at depth 44);
    # contexts sit in reference cycles with their evaluators, so collect
    # them before the next leg allocates.
    import gc
    if not args.skip_ssm:
        log("ssm layer step workload")
        out["ssm_layer_step"] = run_ssm_step()
        gc.collect()
    if not args.skip_bootstrap:
        log("bootstrap workload")
        out["bootstrap"] = run_bootstrap()
        gc.collect()
    decode_ops = None
    if not args.skip_decode:
        log("mamba-2 decode workload")
        out["mamba2_decode"] = run_decode()
        gc.collect()
        if not args.no_cpu_baseline:
            log("mamba-2 decode operation count (for the CPU estimate)")
            decode_ops = count_decode_ops()
            gc.collect()
        log("mamba-2 decode workload, classical-128")
        out["mamba2_decode_classical128"] = run_decode(tokens=3, security="128-classic")
        gc.collect()
    if args.copy_probe:
        log("copy probe")
        copy_probe(F)
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle)")
        out["cpu_baseline"] = cpu_baseline(decode_ops=decode_ops)
    print(json.dumps(out))
    return 0


COPY_PROBE_POLYS, COPY_PROBE_LIMBS = 16, 24
COPY_PROBE_BYTES = COPY_PROBE_POLYS * COPY_PROBE_LIMBS * LIMB


def copy_probe(F) -> None:
    """One k_copy_limbs launch over 16 x 24 limbs (read once, written once)."""
    q = [int(x) for x in ntt_primes(LOG_N, 60, COPY_PROBE_LIMBS)]
    ctx = F.Context(LOG_N, q, [], 1)
    src = ctx.poly(COPY_PROBE_POLYS, COPY_PROBE_LIMBS)
    dst = ctx.poly(COPY_PROBE_POLYS, COPY_PROBE_LIMBS)
    ctx.drop_limbs(src, COPY_PROBE_LIMBS, out=dst)
    ctx.sync()
    ctx.close()


def step_kernel_bytes(L: int, K: int, R: int) -> dict:
    """Bytes each kernel of one rotation step must move (read + write once),
    summed over its launches in the step, for the fused ModUp / ModDown /
    rescale used at this ring dimension.  R hoisted rotations, ne = L + K
    extended limbs, alpha = ceil(L / dnum) limbs per digit:
      ntt_inv_blocks_modup    ModUp's first inverse pass: c1's L limbs read,
                              L written (blocked) and L written as the
                              digits' own limbs;
      k_modup_mid             column stages + conversion of every digit: L
                              read, dnum*(ne-alpha) written;
      ntt_fwd_blocks_modup    last forward pass of the converted limbs:
                              dnum*(ne-alpha) read and written;
      ntt_inv_blocks_ksk      first inverse ModDown pass, fed by the P-limb
                              key inner product: digits dnum*K once per batch,
                              per rotation the key's P limbs dnum*2*K read and
                              2*K written;
      k_moddown_mid           inverse column stages + conversion P -> Q +
                              forward column stages: per rotation 2K read,
                              2L written;
      ntt_fwd_blocks_moddown  last ModDown pass with the Q-limb inner product:
                              digits dnum*L and c0 L once per batch, per
                              rotation y 2L and the key's Q limbs dnum*2*L
                              read, output 2L written;
      rescale (2 polys)       last-limb inverse NTT 2 + 2 per pass, lifted
                              forward column pass 2 read + 2(L-1) written,
                              last pass 2(L-1) read + 2(L-1) of the input
                              read + 2(L-1) written."""
    ne = L + K
    alpha = -(-L // DNUM)
    conv = DNUM * (ne - alpha)
    return {k: v * LIMB for k, v in {
        "ntt_inv_blocks_modup": 3 * L,
        "k_modup_mid": L + conv,
        "ntt_fwd_blocks_modup": 2 * conv,
        "ntt_inv_blocks_ksk": DNUM * K + R * (DNUM * 2 * K + 2 * K),
        "k_moddown_mid": R * (2 * K + 2 * L),
        "ntt_fwd_blocks_moddown": DNUM * L + L + R * (2 * L + DNUM * 2 * L + 2 * L),
        "ntt_inv_blocks_rescale": 4,
        "ntt_inv_cols_rescale": 4,
        "ntt_fwd_cols_rescale": 2 + 2 * (L - 1),
        "ntt_fwd_blocks_rescale": 6 * (L - 1),
    }.items()}


if __name__ == "__main__":
    sys.exit(main())
