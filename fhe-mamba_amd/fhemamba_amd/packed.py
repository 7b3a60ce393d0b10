"""Packed-program executor: a drop-in for the reference's packed_fideslib
(native/fideslib_stage0/src/packed_fideslib.cpp) over this package's CKKS
interface on the GPU.

* Program format `fhemamba-packed-v1` / `-v2` as
  native/fideslib_stage0/include/packed_program.hpp:64-161 reads it (same
  validation, ValueError where the reader throws std::invalid_argument);
  output errors as packed_output_errors (:41-54).
* Node semantics as PackedEvaluator (packed_fideslib.cpp:117-841) in its
  default mode (replicated linear, radix-8 monotone routing): every value
  occupies the leading `size` slots of one ciphertext with zero padding.
* Refresh: before a node runs, a parent whose level plus the node's level
  need would pass the ceiling is masked to its width, scaled by 1 / bound,
  bootstrapped (two passes: the second refreshes the residual times 4096)
  and scaled back (:235-282); the scalings ride on the bootstrap's own
  constants, and the ceiling is L - 3 (42 of 44; the reference's is 39).
* Command line `python -m fhemamba_amd.packed PROGRAM RESULT POLY_TOL
  EXACT_TOL [options]` with the reference's argv and the
  `fhemamba-packed-result-v1` report that src/fhemamba/benchmarks/
  packed.py:188-283 gates on.

Rotation keys are generated on first use for each distinct rotation (one
key switch per rotation) instead of decomposing rotations into the
reference's power-of-two keys: the keys of a program fit in HBM.
"""
from __future__ import annotations

import json
import math
import resource
import sys
import time
from dataclasses import dataclass, field

import numpy as np

from .ptcache import PlaintextCache
from .rotation import bsgs_rotations

try:
    from xxhash import xxh3_128_digest as _digest
except ImportError:  # pragma: no cover - the image ships xxhash
    import hashlib

    def _digest(buf) -> bytes:
        return hashlib.blake2b(buf, digest_size=16).digest()

PACKED_MAX_NODES = 1_000_000
REFRESH_SCALE_BITS = 12          # the reference's 4096 residual scale
CHEB_COEFF_FLOOR = 1e-14         # packed_fideslib.cpp chebyshev(): |c_i| < 1e-14 skipped


# ----------------------------------------------------------------- program
@dataclass
class PackedNode:
    operation: str
    size: int
    parents: list
    data: np.ndarray
    bound: float


@dataclass
class PackedOutput:
    node: int
    polynomial: np.ndarray
    exact: np.ndarray


@dataclass
class PackedProgram:
    magic: str
    slots: int
    bound: float
    nodes: list = field(default_factory=list)
    outputs: list = field(default_factory=list)


class _Tokens:
    def __init__(self, text: str):
        self.items = text.split()
        self.pos = 0

    def has_more(self) -> bool:
        return self.pos < len(self.items)

    def word(self):
        if self.pos >= len(self.items):
            return None
        self.pos += 1
        return self.items[self.pos - 1]

    def int(self):
        w = self.word()
        if w is None:
            return None
        try:
            return int(w)
        except ValueError:
            return None

    def float(self):
        w = self.word()
        if w is None:
            return None
        try:
            return float(w)
        except ValueError:
            return None


def _is_pow2(v: int) -> bool:
    return v > 0 and not v & (v - 1)


def read_packed_program(source) -> PackedProgram:
    """Parse a program from text, bytes or a text stream."""
    if hasattr(source, "read"):
        source = source.read()
    if isinstance(source, bytes):
        source = source.decode()
    t = _Tokens(source)
    magic, slots, bound, nodes, outputs = t.word(), t.int(), t.float(), t.int(), t.int()
    if (outputs is None or magic not in ("fhemamba-packed-v1", "fhemamba-packed-v2")
            or slots < 2 or slots > 32768 or not _is_pow2(slots) or not math.isfinite(bound)
            or bound <= 0 or nodes < 1 or nodes > PACKED_MAX_NODES or outputs < 1
            or outputs > nodes):
        raise ValueError("invalid packed program header")
    v2 = magic == "fhemamba-packed-v2"
    p = PackedProgram(magic, slots, bound)
    for i in range(nodes):
        op, size = t.word(), t.int()
        if op is None or size is None:
            raise ValueError("invalid packed node")
        nb = bound
        if v2:
            nb = t.float()
            if nb is None or not math.isfinite(nb) or nb <= 0 or nb > bound:
                raise ValueError("invalid node refresh bound")
        nparents = t.int()
        if nparents is None or size < 1 or size > slots or nparents < 0 or nparents > 2:
            raise ValueError("invalid packed node")
        parents = []
        for _ in range(nparents):
            par = t.int()
            if par is None or par < 0 or par >= i:
                raise ValueError("invalid packed dependency")
            parents.append(par)
        count = t.int()
        if count is None or count < 0 or count > slots * slots:
            raise ValueError("invalid packed data size")
        data = np.empty(count, dtype=np.float64)
        for j in range(count):
            v = t.float()
            if v is None or not math.isfinite(v):
                raise ValueError("invalid packed constant")
            data[j] = v
        source_op = op in ("input", "public")
        binary = op in ("add", "mul")
        if nparents != (0 if source_op else 2 if binary else 1):
            raise ValueError("wrong operand count")
        in_size = 0 if source_op else p.nodes[parents[0]].size
        valid = False
        if source_op:
            valid = count == size
        elif binary:
            valid = count == 0 and in_size == size and p.nodes[parents[1]].size == size
        elif op in ("addp", "mulp"):
            valid = count == size and in_size == size
        elif op == "linear":
            valid = count == size * in_size
        elif op == "feedback" and v2:
            valid = count == 0 and size == in_size
        elif op == "linear_ref" and v2:
            valid = count == 1 and 0 <= data[0] < i and data[0] == math.floor(data[0])
            if valid:
                w = p.nodes[int(data[0])]
                valid = w.operation == "linear" and w.size == size and \
                    len(w.data) == size * in_size
        elif op == "repeat":
            valid = count == 3 and all(1 <= v <= slots and v == math.floor(v) for v in data)
            if valid:
                rep = int(data[2])
                valid = (v2 or _is_pow2(rep)) and data[0] * data[1] == in_size and \
                    in_size * rep == size
        elif op == "cheb":
            valid = 4 <= count <= 1027 and data[0] < data[1] and in_size == size
        elif op == "sum":
            valid = count == 1 and data[0] >= 1 and data[0] == math.floor(data[0]) and \
                data[0] <= slots and _is_pow2(int(data[0])) and size * data[0] == in_size
        elif op in ("gather", "scatter"):
            valid = count == (size if op == "gather" else in_size)
            limit = in_size if op == "gather" else size
            seen = set()
            for v in data:
                if v < 0 or v >= limit or v != math.floor(v):
                    valid = False
                elif op == "scatter":
                    if int(v) in seen:
                        valid = False
                    seen.add(int(v))
        if not valid:
            raise ValueError("invalid packed operation: " + op)
        p.nodes.append(PackedNode(op, size, parents, data, nb))
    for _ in range(outputs):
        node, size = t.int(), t.int()
        if node is None or size is None or node < 0 or node >= nodes or \
                size != p.nodes[node].size:
            raise ValueError("invalid packed output")
        ref = []
        for _ in range(2 * size):
            v = t.float()
            if v is None or not math.isfinite(v):
                raise ValueError("invalid packed reference")
            ref.append(v)
        p.outputs.append(PackedOutput(node, np.array(ref[:size]), np.array(ref[size:])))
    if t.has_more():
        raise ValueError("trailing packed program data")
    return p


@dataclass
class OutputErrors:
    polynomial: float = 0.0
    exact: float = 0.0
    non_finite: int = 0

    def passes(self, polynomial_tolerance: float, exact_tolerance: float) -> bool:
        return (not self.non_finite and math.isfinite(polynomial_tolerance)
                and math.isfinite(exact_tolerance) and polynomial_tolerance >= 0
                and exact_tolerance >= 0 and self.polynomial <= polynomial_tolerance
                and self.exact <= exact_tolerance)


def packed_output_errors(values, reference: PackedOutput) -> OutputErrors:
    """Max |value - reference| over the output's width (non-finite entries
    counted, not compared)."""
    values = np.asarray(values, dtype=np.float64)
    if len(values) < len(reference.polynomial) or len(reference.exact) != len(reference.polynomial):
        raise ValueError("packed output/reference width mismatch")
    e = OutputErrors()
    for v, p, x in zip(values, reference.polynomial, reference.exact):
        if not (math.isfinite(v) and math.isfinite(p) and math.isfinite(x)):
            e.non_finite += 1
            continue
        e.polynomial = max(e.polynomial, abs(v - p))
        e.exact = max(e.exact, abs(v - x))
    return e


# ----------------------------------------------------------------- plans
def rotation_sum_schedule(count: int):
    """[(offset, accumulated)] such that sum += rot(sum if accumulated else
    input, offset * stride) leaves sum_{k<count} rot(input, k * stride):
    doubling over count's bits (any count, no masks, no depth)."""
    if count <= 0:
        raise ValueError("rotation sum count must be positive")
    steps, filled = [], 1
    for bit in reversed(range(count.bit_length() - 1)):
        steps.append((filled, True))
        filled *= 2
        if count >> bit & 1:
            steps.append((filled, False))
            filled += 1
    return steps


@dataclass(frozen=True)
class ReplicatedShape:
    """out[i] = sum_d W[i][(i + d) mod n] x[(i + d) mod n] with d = j + k r:
    x tiled across a window (window / n copies), the window copied
    `replicas` (+ guard) times, one mask per k serving all r replicas."""
    replicas: int = 1
    window: int = 0
    reps: int = 0
    per_replica: int = 0
    guard: int = 0

    @property
    def baby_step(self) -> int:
        return max(2, int(math.isqrt(self.per_replica)))


def replicated_shape(m: int, n: int, slots: int) -> ReplicatedShape:
    """Largest replica count r <= n whose (r + 1) windows of
    n * ceil((m + r - 1) / n) slots fit; else without the guard window."""
    if m <= 0 or n <= 0 or slots <= 0:
        raise ValueError("replicated matrix dimensions must be positive")
    for r in range(min(n, slots // n - 1), 1, -1):
        window = n * -(-(m + r - 1) // n)
        if (r + 1) * window <= slots:
            return ReplicatedShape(r, window, window // n, -(-n // r), 1)
    window = n * -(-(m + n) // n)
    r = min(n, slots // window)
    if r <= 1:
        return ReplicatedShape()
    return ReplicatedShape(r, window, window // n, -(-n // r), 0)


def replicated_mask(W: np.ndarray, k: int, shape: ReplicatedShape, slots: int,
                    floor: float = 1e-8) -> np.ndarray:
    """Mask of diagonal group k: slot j*window + i + j holds W[i][(i + d) mod n],
    d = j + k r (entries below `floor` in magnitude dropped)."""
    m, n = W.shape
    mask = np.zeros(slots)
    i = np.arange(m)
    for j in range(shape.replicas):
        d = j + k * shape.replicas
        if d >= n:
            continue
        v = W[i, (i + d) % n]
        mask[j * shape.window + i + j] = np.where(np.abs(v) < floor, 0.0, v)
    return mask


def monotone_routing(indices, scatter: bool, bits: int = 3):
    """Stages moving coordinate i by the radix-2^bits digits of its
    displacement (indices[i] - i): ascending digits for a gather
    (compaction), descending for a scatter (expansion), so live coordinates
    never collide.  Each stage maps rotation offset -> source positions."""
    idx = [int(v) for v in indices]
    for i, v in enumerate(idx):
        if v < i or v >= 32768 or (i and v <= idx[i - 1]):
            raise ValueError("routing indices must be strictly increasing")
    pos = list(range(len(idx))) if scatter else list(idx)
    dist = [v - i for i, v in enumerate(idx)]
    top = max(dist) if dist else 0
    shifts = list(range(0, max(top.bit_length(), 1), bits))
    if scatter:
        shifts.reverse()
    stages = []
    for s in shifts:
        stage: dict = {}
        for i in range(len(idx)):
            d = ((dist[i] >> s) & ((1 << bits) - 1)) << s
            stage.setdefault(-d if scatter else d, []).append(pos[i])
            pos[i] += d if scatter else -d
        stages.append(stage)
    return stages


# ----------------------------------------------------------------- evaluator
def default_pt_cache_bytes(device: int | None = None) -> int:
    """Device budget of the evaluator's plaintext cache on `device` (the
    evaluator's context's GPU): 96 GiB, less if the device has under 192
    GiB free when the evaluator is built (the rotation and bootstrapping
    keys, made later, need the rest), and never below an eighth of the free
    memory, so the budget never exceeds what is free.  A
    Mamba-2-130M-shaped decode at N=2^16 encodes ~53 GiB of in_proj /
    out_proj diagonals per token; a budget below its working set evicts each
    diagonal set before its next use (LRU over a cyclic sequence), so every
    token would encode them again."""
    from . import _lib
    free = _lib.device_free_bytes(device)
    cap = 96 << 30
    if free is None:
        return 48 << 30
    return int(max(free // 8, min(cap, free - cap)))


class PackedEvaluator:
    """Evaluates a PackedProgram on a CryptoContext of this package."""

    def __init__(self, cc, keys, slots: int, *, bootstrap_passes: int = 2,
                 refresh_ceiling: int | None = None, replicated_linear: bool = True,
                 trace_levels: bool = False, level_budget=(4, 4), client=None,
                 log=None, pt_cache_bytes: int | None = None, s2c_first: bool = False):
        if bootstrap_passes not in (1, 2):
            raise ValueError("bootstrap passes must be 1 or 2")
        self.cc, self.keys, self.slots = cc, keys, int(slots)
        self.bootstrap_passes = bootstrap_passes
        self.s2c_first = bool(s2c_first)
        # every value here is real: under S2C-first one EvalMod (the real
        # part) is the whole refresh
        cc.EvalBootstrapSetup(list(level_budget), [0, 0], self.slots, s2c_first=self.s2c_first,
                              real_slots=True)
        # deepest level a value may reach and still be masked (one level)
        # and bootstrapped: the bootstrap's input ceiling less one, L - 3
        # (42 for the reference's depth-44 chain; its executor stops at 39,
        # :1132) or, S2C-first, the SlotToCoeff levels lower (:1133)
        self.refresh_ceiling = refresh_ceiling if refresh_ceiling is not None else \
            cc.GetBootstrapInputCeiling() - 1
        self.replicated_linear = replicated_linear
        self.trace_levels = trace_levels
        self.client = client
        self.log = log or (lambda msg: None)
        self._rot_keys: set = set()
        self._masks: dict = {}  # host-side replicated-layout masks by matrix key
        self._pt_cache = PlaintextCache(cc.GetRingDimension(),
                                        pt_cache_bytes if pt_cache_bytes is not None
                                        else default_pt_cache_bytes(
                                            getattr(getattr(cc, "device", None), "device", None)))
        self.stats = dict(ct_ct=0, ct_pt=0, rotations=0, adds=0, bootstraps=0,
                          logical_refreshes=0, bootstrap_seconds=0.0, keygen_seconds=0.0,
                          rotation_keys=0, evaluated_nodes=0)
        self.operation_stats: dict = {}
        self.client_tokens: list = []
        self.client_margins: list = []
        boot_rot = [int(k) % self.slots for k in cc._bootstrapper().rotation_indices()]
        if getattr(keys, "secretKey", None) is None:
            # a server without the secret: every key must have been loaded
            if not cc.HasRotationKeys(boot_rot) or not cc.HasConjugationKey():
                raise ValueError("the loaded key set lacks the bootstrapping keys")
        else:
            t0 = time.perf_counter()
            cc.EvalBootstrapKeyGen(keys.secretKey, self.slots)
            self.stats["keygen_seconds"] += time.perf_counter() - t0
        self._rot_keys.update(boot_rot)

    # ------------------------------------------------------------- primitives
    def _level(self, ct) -> int:
        return ct.GetLevel() + max(0, ct.GetNoiseScaleDeg() - 1)

    def _pad(self, values) -> np.ndarray:
        v = np.zeros(self.slots)
        v[: len(values)] = values
        return v

    def encrypt(self, values):
        pt = self.cc.MakeCKKSPackedPlaintext(self._pad(values), 1, 0, slots=self.slots)
        return self.cc.Encrypt(self.keys.publicKey, pt)

    def _ensure_keys(self, offsets):
        need = sorted({int(o) % self.slots for o in offsets} - {0} - self._rot_keys)
        if need and getattr(self.keys, "secretKey", None) is None:
            if not self.cc.HasRotationKeys(need):
                raise KeyError(f"rotation keys for offsets {need} are not in the loaded key set")
            self._rot_keys.update(need)
        elif need:
            t0 = time.perf_counter()
            self.cc.EvalRotateKeyGen(self.keys.secretKey, need)
            self.stats["keygen_seconds"] += time.perf_counter() - t0
            self.stats["rotation_keys"] += len(need)
            self._rot_keys.update(need)

    def rotate(self, ct, offset: int):
        k = int(offset) % self.slots
        if k == 0:
            return ct
        self._ensure_keys([k])
        self.stats["rotations"] += 1
        return self.cc.EvalRotate(ct, k)

    def rotate_hoisted(self, ct, offsets):
        """Rotations of one ciphertext sharing one ModUp."""
        ks = [int(o) % self.slots for o in offsets]
        todo = sorted({k for k in ks if k})
        out = {0: ct}
        if todo:
            self._ensure_keys(todo)
            self.stats["rotations"] += len(todo)
            pre = self.cc.EvalFastRotationPrecompute(ct)
            for k, r in zip(todo, self.cc.EvalFastRotation(ct, todo, 2 * self.cc.n, pre)):
                out[k] = r
        return [out[k] for k in ks]

    def add(self, a, b):
        self.stats["adds"] += 1
        return self.cc.EvalAdd(a, b)

    def mul(self, a, b):
        self.stats["ct_ct"] += 1
        if a is b:
            return self.cc.EvalSquare(a)
        return self.cc.EvalMult(a, b)

    def scale(self, ct, c: float):
        self.stats["ct_pt"] += 1
        return self.cc.EvalMult(ct, float(c))

    def at_level(self, ct, level: int):
        """ct on `level`'s standard scale (CryptoContext.AlignToLevel)."""
        return self.cc.AlignToLevel(ct, level)

    def plain(self, ct, values, multiply: bool, key=None):
        """ct * values (multiply) or ct + values, the plaintext encoded at
        ct's level.  Plaintexts are cached by `key` (a name for the value
        set) or, without one, by a 128-bit digest of the values: a decode
        meets the same constants (affine maps, masks, biases, taps) at the
        same levels token after token."""
        v = self._pad(values)
        if multiply:
            self.stats["ct_pt"] += 1
            if ct.GetNoiseScaleDeg() >= 2:
                ct = self.cc.Rescale(ct)
            big = float(np.max(np.abs(v))) if len(v) else 0.0
            k = 1
            if big > 4.0:
                # a power-of-two integer part (exact, no level) keeps the
                # encoded values inside the 62-bit coefficient range
                k = 1 << math.ceil(math.log2(big / 2.0))
                ct = self.cc.MultByInteger(ct, k)
                v = v / k
            ck = (key if key is not None else ("mul", _digest(v.data)), ct.GetLevel(), k)
            pt = self._pt_cache.get(ck)
            if pt is None:
                pt = self.cc.MakeCKKSPackedPlaintext(v, 1, ct.GetLevel(), slots=self.slots)
                self._pt_cache.put(ck, pt)
            return self.cc.EvalMult(ct, pt)
        self.stats["adds"] += 1
        # encoded at ct's level and degree: the plaintext EvalAdd would
        # otherwise re-encode from a top-level one
        deg = min(max(int(ct.GetNoiseScaleDeg()), 1), 2)
        ck = (key if key is not None else ("add", _digest(v.data)), ct.GetLevel(), deg)
        pt = self._pt_cache.get(ck)
        if pt is None:
            pt = self.cc.MakeCKKSPackedPlaintext(v, deg, ct.GetLevel(), slots=self.slots)
            self._pt_cache.put(ck, pt)
        return self.cc.EvalAdd(ct, pt)

    def mask(self, ct, size: int):
        return self.plain(ct, np.ones(size), True, key=("ones", size))

    def rotation_sum(self, ct, count: int, stride: int):
        out = ct
        for off, acc in rotation_sum_schedule(count):
            out = self.add(out, self.rotate(out if acc else ct, off * stride))
        return out

    def rotation_sum_many(self, cts, count: int, stride: int):
        """rotation_sum of several ciphertexts in lockstep: each step's
        rotations go out as one batch of key switches (EvalRotateMany)."""
        if len(cts) < 2 or not hasattr(self.cc, "EvalRotateMany"):
            return [self.rotation_sum(c, count, stride) for c in cts]
        base = [self.cc.Rescale(c) if c.GetNoiseScaleDeg() >= 2 else c for c in cts]
        outs = list(base)
        for off, acc in rotation_sum_schedule(count):
            k = (off * stride) % self.slots
            if k == 0:
                outs = [self.add(o, o if acc else b) for o, b in zip(outs, base)]
                continue
            self._ensure_keys([k])
            self.stats["rotations"] += len(outs)
            src = [o if acc else b for o, b in zip(outs, base)]
            src = [self.cc.Rescale(c) if c.GetNoiseScaleDeg() >= 2 else c for c in src]
            rots = self.cc.EvalRotateMany(src, k)
            outs = [self.add(o, r) for o, r in zip(outs, rots)]
        return outs

    # ------------------------------------------------------------- refresh
    def refresh(self, ct, bound: float, support, passes: int | None = None):
        """Mask ct to its support (a width or a 0/1 slot vector; padding is
        never bootstrapped), scale into [-1, 1] by 1 / bound, bootstrap and
        scale back; `passes` (1 or 2) overrides the evaluator's
        bootstrap_passes for this refresh."""
        passes = self.bootstrap_passes if passes is None else passes
        if passes not in (1, 2):
            raise ValueError("bootstrap passes must be 1 or 2")
        t0 = time.perf_counter()
        if isinstance(support, (int, np.integer)):
            x = self.mask(ct, int(support)) if support < self.slots else ct
        else:
            x = self.plain(ct, support, True)
        # 1 / bound and bound ride on the bootstrap's own constants (no
        # level); a power of two keeps the SlotToCoeff diagonals the same
        # for every bound (it goes into EvalMod's integer gain or the last
        # group's constant), at most one bit of the range given up
        bound = 2.0 ** math.ceil(math.log2(max(float(bound), 2.0 ** -30)))
        out = self.cc.EvalBootstrap(x, passes, REFRESH_SCALE_BITS, scale=bound)
        self.stats["bootstraps"] += passes
        self.stats["logical_refreshes"] += 1
        self.stats["bootstrap_seconds"] += time.perf_counter() - t0
        return out

    def refresh_many(self, cts, bound: float, support, passes: int | None = None) -> list:
        """refresh of every ciphertext of `cts` (one bound and support)
        through the context's multi-ciphertext bootstrap when it has one,
        else one at a time.  Under S2C-first the (real) values go in pairs,
        as the reference's complex state pairing does (maybe_bootstrap_pair,
        stage1_mamba2_decode_fideslib.cpp:2298-2330): c = (a + i b) / 2, the
        1/2 riding on the support mask, one complex-slot bootstrap per pair
        (both EvalMods; ~1.5 real ones), then a = c + conj(c) and b = -i (c
        - conj(c)); the pairs' stages in step."""
        cts = list(cts)
        many = getattr(self.cc, "EvalBootstrapMany", None)
        if len(cts) <= 1 or many is None:
            return [self.refresh(ct, bound, support, passes) for ct in cts]
        passes = self.bootstrap_passes if passes is None else passes
        if passes not in (1, 2):
            raise ValueError("bootstrap passes must be 1 or 2")
        t0 = time.perf_counter()
        pair = self.s2c_first
        if isinstance(support, (int, np.integer)):
            if support < self.slots or pair:
                sup = np.zeros(self.slots)
                sup[: int(support)] = 1.0
                xs = [self.plain(ct, sup * (0.5 if pair else 1.0), True) for ct in cts]
            else:
                xs = cts
        else:
            xs = [self.plain(ct, np.asarray(support) * (0.5 if pair else 1.0), True)
                  for ct in cts]
        bound = 2.0 ** math.ceil(math.log2(max(float(bound), 2.0 ** -30)))
        if not pair:
            outs = many(xs, passes, REFRESH_SCALE_BITS, scale=bound)
            self.stats["bootstraps"] += passes * len(cts)
        else:
            cc, half = self.cc, self.cc.GetRingDimension() // 2
            packed = [cc.EvalAdd(a, cc.MultByMonomial(b, half)) for a, b in zip(xs[0::2], xs[1::2])]
            if len(xs) % 2:
                packed.append(xs[-1])
            got = many(packed, passes, REFRESH_SCALE_BITS, scale=bound, real_slots=False)
            conj = cc.EvalConjugateMany(got)
            outs = []
            for c, cj in zip(got, conj):
                outs.append(cc.EvalAdd(c, cj))
                outs.append(cc.MultByMonomial(cc.EvalSub(c, cj), 3 * half))
            outs = outs[: len(cts)]
            self.stats["bootstraps"] += passes * len(packed)
        self.stats["logical_refreshes"] += len(cts)
        self.stats["bootstrap_seconds"] += time.perf_counter() - t0
        return outs

    # ------------------------------------------------------------- node kinds
    def transform(self, x, masks: dict, key=None):
        """sum over offsets of rot(x, offset) * mask.  Offsets on an
        arithmetic progression (8 or more) go through the baby-step
        giant-step transform (about 2 sqrt(count) rotations and keys, as
        the reference's plan_packed_diagonals, include/packed_routing.hpp:
        23-45); others are hoisted rotations of x.  `key` names the mask set
        for the plaintext cache."""
        if not masks:
            return self.scale(x, 0.0)
        offs = sorted(masks)
        step = offs[1] - offs[0] if len(offs) > 1 else 0
        if len(offs) >= 8 and step and all(b - a == step for a, b in zip(offs, offs[1:])):
            return self._transform_bsgs(x, offs, step, masks, key)
        rots = self.rotate_hoisted(x, offs)
        out = None
        for off, r in zip(offs, rots):
            term = self.plain(r, masks[off], True)
            out = term if out is None else self.add(out, term)
        return out

    def _encode_rows(self, rows, level: int) -> list:
        """Degree-1 plaintexts of the slot vectors `rows` at `level`, in one
        batched encode where the context offers it."""
        many = getattr(self.cc, "MakeCKKSPackedPlaintexts", None)
        if many is not None:
            return many(rows, 1, level, slots=self.slots)
        return [self.cc.MakeCKKSPackedPlaintext(r, 1, level, slots=self.slots) for r in rows]

    def _transform_bsgs(self, x, offs, step, masks, key):
        rows = len(offs)
        b = max(2, 1 << round(math.log2(math.sqrt(rows))))
        if x.GetNoiseScaleDeg() >= 2:
            x = self.cc.Rescale(x)
        level = x.GetLevel()
        ck = None if key is None else (key, "bsgs", level)
        pts = self._pt_cache.get(ck) if ck else None
        if pts is None:
            pts = self._encode_rows([np.roll(masks[o], (k // b) * b * step)
                                     for k, o in enumerate(offs)], level)
            if ck:
                self._pt_cache.put(ck, pts)
        giants = -(-rows // b)
        self._ensure_keys(bsgs_rotations(rows, b, step, offs[0]))
        self.stats["rotations"] += (min(b, rows) - 1) + (giants - 1) + (1 if offs[0] % self.slots else 0)
        self.stats["ct_pt"] += rows
        out = x.Clone()
        self.cc.LinearTransformInPlace(out, rows, b, pts, step % self.slots, offs[0] % self.slots)
        return out

    def gather(self, x, indices, size: int, scatter: bool, bound: float, width: int):
        idx = [int(v) for v in indices]
        if scatter and idx == list(range(len(idx))):
            return x
        monotone = all(idx[i] > idx[i - 1] for i in range(1, len(idx)))
        offsets = {v - i for i, v in enumerate(idx)}
        if self.replicated_linear and monotone and len(offsets) > 32:
            out = x
            for stage in monotone_routing(idx, scatter):
                if self._level(out) + 3 > self.refresh_ceiling:
                    out = self.refresh(out, bound, max(size, width))
                # rot(x * source mask, o) = rot(x, o) * destination mask: the
                # stage's rotations of one ciphertext share one ModUp
                masks = {}
                for off, positions in stage.items():
                    dest = np.asarray(positions) - off
                    if dest.min() < 0 or dest.max() >= self.slots:
                        raise ValueError("routing stage leaves the slot range")
                    masks.setdefault(off, np.zeros(self.slots))[dest] = 1.0
                out = self.transform(out, masks)
            return out
        masks: dict = {}
        for i, v in enumerate(idx):
            src, dst = (i, v) if scatter else (v, i)
            masks.setdefault(src - dst, np.zeros(self.slots))[dst] = 1.0
        return self.transform(x, masks)

    def linear(self, x, W: np.ndarray, key):
        m, n = W.shape
        shape = replicated_shape(m, n, self.slots) if self.replicated_linear and \
            m + n <= self.slots else ReplicatedShape()
        if shape.replicas > 1:
            ext = self.rotation_sum(x, shape.reps, -n)
            rep = self.rotation_sum(ext, shape.replicas + shape.guard, -shape.window)
            self.cc.RescaleInPlace(rep)
            b = min(shape.baby_step, shape.per_replica)
            stride = shape.replicas
            cache_key = (key, "replicated", rep.GetLevel())
            pts = self._pt_cache.get(cache_key)
            if pts is None:
                pts = self._encode_rows(self._replicated_masks(W, shape, b, stride, key),
                                        rep.GetLevel())
                self._pt_cache.put(cache_key, pts)
            self._ensure_keys(bsgs_rotations(shape.per_replica, b, stride))
            giants = -(-shape.per_replica // b)
            self.stats["rotations"] += (b - 1) + (giants - 1)
            self.stats["ct_pt"] += shape.per_replica
            out = rep.Clone()
            self.cc.LinearTransformInPlace(out, shape.per_replica, b, pts, stride, 0)
            out = self.rotation_sum(out, shape.replicas, shape.window + 1)
            return self.mask(out, m)
        masks: dict = {}
        for i in range(m):
            for j in range(n):
                if W[i, j] != 0:
                    masks.setdefault(j - i, np.zeros(self.slots))[i] = W[i, j]
        return self.transform(x, masks)

    def _replicated_masks(self, W, shape, b: int, stride: int, key):
        """The replicated layout's diagonal-group masks, each rolled for its
        giant step.  They do not depend on the level, while their encodings
        do: a matrix met at a new level (the carried state moves the
        projections' levels from token to token) re-encodes from these
        instead of rebuilding them."""
        ck = None if key is None else (key, shape, b, stride)
        masks = self._masks.get(ck) if ck is not None else None
        if masks is None:
            masks = [np.roll(replicated_mask(W, k, shape, self.slots), (k // b) * b * stride)
                     for k in range(shape.per_replica)]
            if ck is not None:
                self._masks[ck] = masks
        return masks

    def chebyshev(self, x, node: PackedNode):
        from .ckks_probes import chebyshev_ps
        lo, hi = float(node.data[0]), float(node.data[1])
        size = node.size
        u = self.plain(x, np.full(size, 2.0 / (hi - lo)), True, key=("cheb-a", lo, hi, size))
        u = self.plain(u, np.full(size, -(lo + hi) / (hi - lo)), False)
        coeffs = [float(c) for c in node.data[2:]]
        counting = _CountingContext(self.cc, self.stats)
        p = chebyshev_ps(counting, u, coeffs, CHEB_COEFF_FLOOR, lambda v: self.scale(u, 0.0))
        return self.mask(p, size)

    # ------------------------------------------------------------- program
    def _need(self, node: PackedNode) -> int:
        if node.operation == "cheb":
            return max(1, math.ceil(math.log2(len(node.data) - 2))) + 5
        return 3

    def evaluate(self, program: PackedProgram):
        nodes = program.nodes
        last_use = [-1] * len(nodes)
        for i, nd in enumerate(nodes):
            for par in nd.parents:
                last_use[par] = i
        pinned = {o.node for o in program.outputs}
        values: list = [None] * len(nodes)
        t_start = time.perf_counter()
        for i, nd in enumerate(nodes):
            t0 = time.perf_counter()
            b0, s0 = self.stats["bootstraps"], self.stats["bootstrap_seconds"]
            op = nd.operation
            need = self._need(nd)
            for par in nd.parents:
                if op != "feedback" and self._level(values[par]) + need > self.refresh_ceiling:
                    values[par] = self.refresh(values[par], nodes[par].bound, nodes[par].size)
            x = values[nd.parents[0]] if nd.parents else None
            if self.trace_levels:
                self.log(f"level_input node={i} op={op} parents=" + ",".join(
                    f"{p}:{values[p].GetLevel()}" for p in nd.parents))
            if op in ("input", "public"):
                out = self.encrypt(nd.data)
            elif op == "feedback":
                if self.client is None:
                    raise RuntimeError("client feedback requires --client-head")
                out = self.encrypt(self.client(self, i, x))
            elif op == "add":
                out = self.add(x, values[nd.parents[1]])
            elif op == "mul":
                y = values[nd.parents[1]]
                out = self.mul(x, x if nd.parents[0] == nd.parents[1] else y)
            elif op in ("addp", "mulp"):
                out = self.plain(x, nd.data, op == "mulp")
            elif op in ("gather", "scatter"):
                out = self.gather(x, nd.data, nd.size, op == "scatter", nd.bound,
                                  nodes[nd.parents[0]].size)
            elif op in ("linear", "linear_ref"):
                src = i if op == "linear" else int(nd.data[0])
                cols = nodes[nd.parents[0]].size
                W = nodes[src].data.reshape(nd.size, cols)
                out = self.linear(x, W, ("linear", src))
            elif op == "cheb":
                out = self.chebyshev(x, nd)
            elif op == "repeat":
                outer, inner, rep = (int(v) for v in nd.data)
                dest = [g * inner * rep + j for g in range(outer) for j in range(inner)]
                out = self.gather(x, dest, nd.size, True, nd.bound, nodes[nd.parents[0]].size)
                out = self.rotation_sum(out, rep, -inner)
            elif op == "sum":
                width = int(nd.data[0])
                out = x
                step = 1
                while step < width:
                    out = self.add(out, self.rotate(out, step))
                    step *= 2
                out = self.gather(out, [j * width for j in range(nd.size)], nd.size, False,
                                  nd.bound, nodes[nd.parents[0]].size)
            else:
                raise ValueError(f"unknown packed operation {op}")
            values[i] = out
            for par in nd.parents:
                if last_use[par] == i and par not in pinned:
                    values[par] = None
            self.stats["evaluated_nodes"] += 1
            st = self.operation_stats.setdefault(op, dict(nodes=0, seconds=0.0,
                                                          bootstrap_seconds=0.0, bootstraps=0))
            st["nodes"] += 1
            st["seconds"] += time.perf_counter() - t0
            st["bootstrap_seconds"] += self.stats["bootstrap_seconds"] - s0
            st["bootstraps"] += self.stats["bootstraps"] - b0
            if self.trace_levels:
                self.log(f"level_output node={i} level={out.GetLevel()} "
                         f"degree={out.GetNoiseScaleDeg()}")
            done = i + 1
            if done % 10 == 0 or done == len(nodes):
                el = time.perf_counter() - t_start
                self.log(f"node={done}/{len(nodes)} op={op} seconds={el:.3f} "
                         f"eta_seconds={el * (len(nodes) - done) / done:.3f} "
                         f"bootstraps={self.stats['bootstraps']}")
        return [values[o.node] for o in program.outputs]

    def decrypt(self, ct, size: int) -> np.ndarray:
        pt = self.cc.Decrypt(ct, self.keys.secretKey)
        pt.SetLength(size)
        return np.asarray(pt.GetRealPackedValue(), dtype=np.float64)[:size]


class _CountingContext:
    """Forwards to the CryptoContext, counting products and additions."""

    def __init__(self, cc, stats):
        self._cc, self._stats = cc, stats

    def EvalMult(self, a, b):  # noqa: N802
        self._stats["ct_pt" if isinstance(b, (int, float)) else "ct_ct"] += 1
        return self._cc.EvalMult(a, b)

    def EvalAdd(self, a, b):  # noqa: N802
        self._stats["adds"] += 1
        return self._cc.EvalAdd(a, b)

    def EvalSub(self, a, b):  # noqa: N802
        self._stats["adds"] += 1
        return self._cc.EvalSub(a, b)

    def __getattr__(self, name):
        # Rescale, EvalLinearWSum and the rest go straight through
        return getattr(self._cc, name)


# ----------------------------------------------------------------- client head
class GenerationClient:
    """Client side of feedback nodes (packed_fideslib.cpp:843-880): decrypts
    the final hidden vector, picks the greedy token from a vocabulary head
    (uint32 vocabulary, uint32 width, vocabulary x width float32 LE) and
    returns that token's row as the next embedding."""

    def __init__(self, path: str):
        with open(path, "rb") as f:
            raw = f.read()
        if len(raw) < 8:
            raise ValueError("invalid client vocabulary head")
        vocab, width = np.frombuffer(raw[:8], dtype="<u4")
        vocab, width = int(vocab), int(width)
        if vocab < 2 or vocab > 262144 or width < 1 or width > 8192 or vocab * width > 268435456:
            raise ValueError("invalid client vocabulary head")
        if len(raw) != 8 + 4 * vocab * width:
            raise ValueError("invalid client head length")
        w = np.frombuffer(raw[8:], dtype="<f4").astype(np.float64).reshape(vocab, width)
        if not np.isfinite(w).all():
            raise ValueError("nonfinite client head")
        self.vocabulary, self.width, self.weights = vocab, width, w
        self.tokens: list = []
        self.margins: list = []

    def select(self, hidden) -> np.ndarray:
        h = np.asarray(hidden, dtype=np.float64)
        if len(h) < self.width:
            raise ValueError("client hidden width mismatch")
        if not np.isfinite(h[: self.width]).all():
            raise RuntimeError("nonfinite client output")
        logits = self.weights @ h[: self.width]
        best = int(np.argmax(logits))
        top2 = np.sort(logits)[-2:] if self.vocabulary > 1 else logits
        self.tokens.append(best)
        self.margins.append(float(top2[-1] - top2[0]))
        return self.weights[best].copy()


# ----------------------------------------------------------------- command line
USAGE = ("usage: python -m fhemamba_amd.packed PROGRAM RESULT POLY_TOL EXACT_TOL "
         "[--direct-linear] [--bootstrap-passes 1|2] [--trace-levels] "
         "[--client-head FILE] [reference performance options]")
# Reference options that tune FIDESlib's internals (plaintext caching and
# upload paths, in-place scratch reuse, refresh planning, rotation
# decomposition); accepted and recorded, they do not change the result
# beyond CKKS precision.
_FLAG_OPTIONS = {
    "--legacy-routing", "--planned-refresh", "--batch-refresh", "--merge-refresh-correction",
    "--profile-evaluation", "--inplace-ops", "--naf-rotations", "--reuse-dead-inputs",
    "--reuse-public-ciphertexts", "--compact-weights", "--cache-plaintexts",
    "--indexed-mask-cache", "--prefetch-plaintexts", "--fast-plaintext-upload",
    "--direct-plaintext-upload", "--gpu-plaintext-ntt", "--move-plaintext-coefficients",
    "--borrow-plaintext-upload", "--bsgs-routing-stages", "--frontier-refresh",
    "--gpu-plaintext-rns", "--gpu-addend-rns", "--gpu-plaintext-fft", "--batch-plaintext-rns",
    "--fuse-plaintext-rns-ntt", "--hoist-rotations", "--share-chebyshev",
}
_VALUE_OPTIONS = {"--plaintext-cache-capacity", "--prefetch-workers", "--frontier-live-limit",
                  "--security-digits"}
_UNSUPPORTED = {"--gpu-dual-ring", "--diagnostic-reference",
                "--diagnostic-output", "--diagnostic-refresh-pair"}


def parse_args(argv):
    if len(argv) < 4:
        raise ValueError(USAGE)
    opts = dict(program=argv[0], result=argv[1], direct_linear=False, bootstrap_passes=2,
                trace_levels=False, client_head=None, security="not-set", s2c_first=False,
                accepted=[])
    poly_tol, exact_tol = float(argv[2]), float(argv[3])
    i = 4
    while i < len(argv):
        a = argv[i]
        if a == "--direct-linear":
            opts["direct_linear"] = True
        elif a == "--trace-levels":
            opts["trace_levels"] = True
        elif a == "--s2c-first":
            opts["s2c_first"] = True
        elif a == "--bootstrap-passes" and i + 1 < len(argv):
            i += 1
            opts["bootstrap_passes"] = int(argv[i])
            if opts["bootstrap_passes"] not in (1, 2):
                raise ValueError("bootstrap passes must be 1 or 2")
        elif a == "--client-head" and i + 1 < len(argv):
            i += 1
            opts["client_head"] = argv[i]
        elif a == "--security" and i + 1 < len(argv):
            i += 1
            opts["security"] = argv[i]
        elif a in _FLAG_OPTIONS:
            opts["accepted"].append(a)
        elif a in _VALUE_OPTIONS and i + 1 < len(argv):
            opts["accepted"].append(f"{a} {argv[i + 1]}")
            i += 1
        elif a in _UNSUPPORTED:
            raise ValueError(f"packed option {a} is not supported by this executor")
        else:
            raise ValueError("unknown packed option: " + a)
        i += 1
    if opts["security"] not in ("not-set", "128-classic"):
        raise ValueError("security must be not-set or 128-classic")
    # refresh-planning rules of packed_fideslib.cpp:1013-1017
    acc = set(opts["accepted"])
    if "--batch-refresh" in acc and ("--planned-refresh" not in acc or
                                     opts["bootstrap_passes"] != 2):
        raise ValueError("batch refresh requires planned refresh and two bootstrap passes")
    if opts["s2c_first"] and "--batch-refresh" not in acc:
        raise ValueError("S2C-first requires planned two-pass batch refresh")
    # --security-digits: HYBRID digits of the classical-128 context, 1..16,
    # only with 128-classic (packed_fideslib.cpp:913-914, :974, :991-992)
    digits = [a for a in opts["accepted"] if a.startswith("--security-digits ")]
    opts["accepted"] = [a for a in opts["accepted"] if not a.startswith("--security-digits ")]
    opts["security_digits"] = int(digits[-1].split()[1]) if digits else 4
    if not 1 <= opts["security_digits"] <= 16 or (digits and opts["security"] != "128-classic"):
        raise ValueError("--security-digits must be 1..16 and requires --security 128-classic")
    if not (math.isfinite(poly_tol) and math.isfinite(exact_tol)) or poly_tol <= 0 or \
            exact_tol <= 0:
        raise ValueError("invalid error tolerance")
    opts["poly_tol"], opts["exact_tol"] = poly_tol, exact_tol
    return opts


# Classical-128 as the reference executor sets it up (packed_fideslib.cpp:
# 1042, 1060-1075): ring 2^17, full packing (65536 slots), uniform ternary,
# HEStd_128_classic and `security_digits` HYBRID digits (default 4), the
# audit required before any key is made.
CLASSICAL128 = dict(ring_dim=131072, dnum=4, security="128-classic")


def build_context(slots: int, *, ring_dim: int = 65536, depth: int = 44, scale_bits: int = 59,
                  first_mod_bits: int = 60, dnum: int = 3, seed=None, secret_dist=None,
                  security: str = "not-set"):
    """The reference executor's context (packed_fideslib.cpp:1060-1083):
    uniform ternary (unless `secret_dist` says otherwise), FLEXIBLEAUTO,
    HYBRID, depth 44, 59-bit scale, 60-bit first prime, dnum 3, batch =
    program slots, security not set; with security "128-classic" the
    security level is HEStd_128_classic and the context must pass the
    classical-128 audit (RequireClassical128) before keys are generated."""
    from . import ckks
    if security not in ("not-set", "128-classic"):
        raise ValueError("security must be not-set or 128-classic")
    p = ckks.CCParamsCKKSRNS()
    p.SetSecurityLevel(ckks.SecurityLevel.HEStd_128_classic if security == "128-classic"
                       else ckks.SecurityLevel.HEStd_NotSet)
    p.SetSecretKeyDist(secret_dist or ckks.SecretKeyDist.UNIFORM_TERNARY)
    p.SetRingDim(ring_dim)
    p.SetBatchSize(slots)
    p.SetMultiplicativeDepth(depth)
    p.SetScalingModSize(scale_bits)
    p.SetFirstModSize(first_mod_bits)
    p.SetScalingTechnique(ckks.ScalingTechnique.FLEXIBLEAUTO)
    p.SetKeySwitchTechnique(ckks.KeySwitchTechnique.HYBRID)
    p.SetNumLargeDigits(dnum)
    cc = ckks.GenCryptoContext(p, seed=seed)
    if security == "128-classic":
        cc.RequireClassical128()
    for f in (ckks.PKESchemeFeature.PKE, ckks.PKESchemeFeature.KEYSWITCH,
              ckks.PKESchemeFeature.LEVELEDSHE, ckks.PKESchemeFeature.ADVANCEDSHE,
              ckks.PKESchemeFeature.FHE):
        cc.Enable(f)
    keys = cc.KeyGen()
    cc.EvalMultKeyGen(keys.secretKey)
    return cc, keys


def run(program: PackedProgram, opts: dict, *, context_args=None, log=print) -> tuple[dict, bool]:
    """Evaluate, decrypt and compare; returns (report, passed)."""
    t_setup = time.perf_counter()
    args = dict(context_args or {})
    classical = opts.get("security") == "128-classic"
    if classical:
        # full packing, as the reference's S2C-first circuit requires
        # (packed_fideslib.cpp:1040-1042); node widths stay the program's
        program.slots = 65536
        args.update(CLASSICAL128, dnum=opts.get("security_digits", 4))
    if opts.get("s2c_first") and program.slots != args.get("ring_dim", 65536) // 2:
        raise ValueError("S2C-first requires full packing (program slots = ring dimension / 2)")
    cc, keys = build_context(program.slots, **args)
    audit = cc.SecurityAudit() if classical else None
    if classical and opts.get("result"):
        with open(opts["result"] + ".parameters.json", "w") as f:
            f.write(json.dumps(audit) + "\n")
        log(f"classical128 ring={audit['ring_dimension']} QP_bits={audit['qp_bits']} "
            f"bound={audit['guideline_max_qp_bits']} digits={audit['hybrid_digits']}")
    client = GenerationClient(opts["client_head"]) if opts.get("client_head") else None
    if client is not None and program.nodes[program.outputs[-1].node].size != client.width:
        raise ValueError("client head and final hidden width mismatch")
    feedback_outputs = []
    positions = {o.node: k for k, o in enumerate(program.outputs)}
    for nd in program.nodes:
        if nd.operation == "feedback":
            feedback_outputs.append(positions.get(nd.parents[0], -1))

    def client_step(ev, node_index, hidden):
        values = ev.decrypt(hidden, client.width)
        k = feedback_outputs[len(client.tokens)]
        if k >= 0:
            e = packed_output_errors(values, program.outputs[k])
            if not e.passes(opts["poly_tol"], opts["exact_tol"]):
                raise RuntimeError("client hidden fails reference tolerance before token "
                                   f"{len(client.tokens) + 1}")
        return client.select(values)

    ev = PackedEvaluator(cc, keys, program.slots, bootstrap_passes=opts["bootstrap_passes"],
                         replicated_linear=not opts["direct_linear"],
                         trace_levels=opts["trace_levels"],
                         client=client_step if client else None, log=log,
                         s2c_first=opts.get("s2c_first", False))
    setup_s = time.perf_counter() - t_setup
    log(f"setup_seconds={setup_s}")
    t0 = time.perf_counter()
    outs = ev.evaluate(program)
    cc.device.sync()
    eval_s = time.perf_counter() - t0
    if client is not None:
        client.select(ev.decrypt(outs[-1], client.width))
    poly_err = exact_err = 0.0
    non_finite = 0
    per_output = []
    for o, ct in zip(program.outputs, outs):
        e = packed_output_errors(ev.decrypt(ct, len(o.polynomial)), o)
        non_finite += e.non_finite
        poly_err, exact_err = max(poly_err, e.polynomial), max(exact_err, e.exact)
        per_output.append({"polynomial": float(e.polynomial), "exact": float(e.exact)})
    poly_err, exact_err = float(poly_err), float(exact_err)
    passed = bool(non_finite == 0 and poly_err <= opts["poly_tol"] and
                  exact_err <= opts["exact_tol"])
    s = ev.stats
    report = {
        "schema": "fhemamba-packed-result-v1",
        "backend": "fhemamba_amd (MI355X HIP)",
        "encrypted": True,
        "security": opts["security"],
        "passed": passed,
        "slots": program.slots,
        "payload_slots": program.slots,
        "ring_dimension": cc.GetRingDimension(),
        "depth": len(cc.GetModuli()[0]) - 1,
        "scale_bits": round(math.log2(cc.GetScalingFactorReal(0))),
        "refresh_ring_dimension": cc.GetRingDimension(),
        "security_audit": audit,
        "gpu_dual_ring": False,
        "nodes": len(program.nodes),
        "setup_seconds": setup_s,
        "evaluated_nodes": s["evaluated_nodes"],
        "eval_seconds": eval_s,
        "bootstrap_seconds": s["bootstrap_seconds"],
        "bootstraps": s["bootstraps"],
        "logical_refreshes": s["logical_refreshes"],
        "ct_ct_mul": s["ct_ct"],
        "ct_pt_mul": s["ct_pt"],
        "rotations": s["rotations"],
        "adds": s["adds"],
        "rotation_keys_generated": s["rotation_keys"],
        "keygen_seconds": s["keygen_seconds"],
        "linear_method": "replicated-bsgs" if ev.replicated_linear else "direct",
        "routing_method": "radix8-direct32" if ev.replicated_linear else "direct",
        "refresh_policy": "baseline",
        "refresh_ceiling": ev.refresh_ceiling,
        "s2c_first": ev.s2c_first,
        "bootstrap_passes": ev.bootstrap_passes,
        "accepted_options": opts.get("accepted", []),
        "max_abs_error_vs_polynomial": poly_err,
        "max_abs_error_vs_exact": exact_err,
        "non_finite": non_finite,
        "polynomial_tolerance": opts["poly_tol"],
        "exact_tolerance": opts["exact_tol"],
        "peak_rss_gib": resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / (1024.0 * 1024.0),
        "per_output_errors": per_output,
        "diagnostic_only": False,
        "evaluation_decryptions": 0,
        "client_output_decrypt_count": len(client.tokens) if client else 0,
        "generated_token_ids": list(client.tokens) if client else [],
        "client_logit_margins": list(client.margins) if client else [],
        "operation_stats": ev.operation_stats,
        "scope": ("packed feasibility; inline client fixture" if client is None else
                  "encrypted backbone with inline client vocabulary head and actual greedy "
                  "feedback"),
    }
    log(f"passed={int(passed)} polynomial_error={poly_err} exact_error={exact_err} "
        f"eval_seconds={eval_s}")
    return report, passed


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    try:
        opts = parse_args(argv)
        with open(opts["program"]) as f:
            program = read_packed_program(f)
        report, passed = run(program, opts)
        with open(opts["result"], "w") as f:
            f.write(json.dumps(report, indent=None) + "\n")
        return 0 if passed else 1
    except Exception as exc:  # noqa: BLE001 - the reference reports every failure as exit 2
        print(exc, file=sys.stderr)
        return 2


if __name__ == "__main__":
    sys.exit(main())
