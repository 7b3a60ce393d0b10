"""CKKS circuit helpers with the interface of src/fhemamba/ckks_probes.py.

CkksPrimitives drives any object with the OpenFHE CryptoContext surface
(by default this package's fhemamba_amd.ckks on the GPU); the helpers below
follow src/fhemamba/ckks_probes.py:10-164 so that the same circuits issue
the same sequence of homomorphic operations:
  * floor_coeffs / affine / cheb_eval64 / ceil_log2 (:13-31);
  * cheb_baby_size: 2^ceil(levels / 2), levels = max(1, ceil(log2(d + 1)))
    (:34-36);
  * cheb_ps_depth: the level ledger of the Paterson-Stockmeyer recursion
    (:39-66);
  * eval_chebyshev: Paterson-Stockmeyer over Chebyshev polynomials with
    T_2i = 2 T_i^2 - 1, T_2i+1 = 2 T_i+1 T_i - T_1 and the split
    p = a' + T_k * b~ (:107-155);
  * newton_refine: y <- 1.5 y + (-v/2) y^3 (:157-164);
  * build_toy_context (:167-201), TOY security (HEStd_NotSet).
"""
from __future__ import annotations

from typing import Sequence

import numpy as np

CHEB_COEFF_FLOOR = 1e-12


def floor_coeffs(coeffs, threshold: float = CHEB_COEFF_FLOOR) -> list[float]:
    """Zero every coefficient below the floor (in magnitude)."""
    return [float(c) if abs(float(c)) >= threshold else 0.0 for c in coeffs]


def affine(lo: float, hi: float) -> tuple[float, float]:
    """(a, b) such that a * x + b maps [lo, hi] onto [-1, 1]."""
    width = hi - lo
    return 2.0 / width, -(hi + lo) / width


def cheb_eval64(coeffs: Sequence[float], u: np.ndarray) -> np.ndarray:
    return np.polynomial.chebyshev.chebval(u, np.asarray(coeffs, dtype=np.float64))


def ceil_log2(value: int) -> int:
    """Smallest e >= 0 with 2^e >= value."""
    e = 0
    while (1 << e) < value:
        e += 1
    return e


def cheb_baby_size(degree: int) -> int:
    levels = max(1, ceil_log2(degree + 1))
    return 1 << ((levels + 1) // 2)


def _giant_split(n: int, m: int) -> int:
    """Smallest k = m * 2^j with 2k - 1 >= n."""
    k = m
    while 2 * k - 1 < n:
        k *= 2
    return k


def cheb_ps_depth(degree: int, baby: int | None = None) -> int:
    """Multiplicative depth the Paterson-Stockmeyer evaluation spends
    (baby-step size `baby`, default cheb_baby_size(degree))."""
    m = baby or cheb_baby_size(degree)
    memo: dict[int, int] = {}

    def t_depth(i: int) -> int:
        if i <= 1:
            return 0
        if i not in memo:
            if i % 2 == 0:
                memo[i] = t_depth(i // 2) + 1
            else:
                memo[i] = max(t_depth(i // 2), t_depth(i // 2 + 1)) + 1
        return memo[i]

    def depth(n: int) -> int:
        if n == 0:
            return 0
        if n < m:
            return 1 + max(t_depth(i) for i in range(1, n + 1))
        k = _giant_split(n, m)
        return max(depth(k - 1), 1 + max(t_depth(k), depth(n - k)))

    return depth(degree)


def _mult_many(cc, pairs):
    """EvalMult of every pair, relinearized together when the context has
    EvalMultMany (independent products of one circuit step), else one
    EvalMult each; the same ciphertexts either way."""
    many = getattr(cc, "EvalMultMany", None)
    if many is not None and len(pairs) > 1:
        return many(pairs)
    return [cc.EvalMult(a, b) for a, b in pairs]


def _t_depth(i: int, memo: dict) -> int:
    if i <= 1:
        return 0
    if i not in memo:
        if i % 2 == 0:
            memo[i] = _t_depth(i // 2, memo) + 1
        else:
            memo[i] = max(_t_depth(i // 2, memo), _t_depth(i // 2 + 1, memo)) + 1
    return memo[i]


class ChebBasis:
    """T_i(u) built on demand from T_1 = u by T_2j = 2 T_j^2 - 1 and
    T_2j+1 = 2 T_j+1 T_j - u, each kept once (series of one input may share
    it).  Backends with Rescale keep each basis polynomial rescaled once (it
    is multiplied many times)."""

    def __init__(self, cc, u):
        self.cc, self.u = cc, u
        self.settle = getattr(cc, "Rescale", None) or (lambda ct: ct)
        self.cache = {1: u}

    @staticmethod
    def _operands(i: int) -> tuple:
        return (i // 2, i // 2) if i % 2 == 0 else (i // 2 + 1, i // 2)

    def _unsettled(self, i: int, product):
        cc = self.cc
        return cc.EvalSub(cc.EvalAdd(product, product), 1.0 if i % 2 == 0 else self.u)

    def _finish(self, i: int, product):
        self.cache[i] = self.settle(self._unsettled(i, product))

    def __call__(self, i: int):
        if i not in self.cache:
            a, b = self._operands(i)
            ta = self(a)
            self._finish(i, self.cc.EvalMult(ta, ta if a == b else self(b)))
        return self.cache[i]

    @staticmethod
    def build_many(requests) -> None:
        """For (basis, indices) pairs: every T_i the indices need, by
        increasing depth, the products of one depth over all the bases
        multiplied together (_mult_many) and rescaled together (RescaleMany,
        where the context has it); each T_i is the value __call__
        computes."""
        memo: dict = {}
        todo = []
        for basis, indices in requests:
            need, stack = set(), list(indices)
            while stack:
                i = stack.pop()
                if i <= 1 or i in need or i in basis.cache:
                    continue
                need.add(i)
                stack.extend(basis._operands(i))
            todo.extend((basis, i) for i in need)
        if not todo:
            return
        for d in range(1, max(_t_depth(i, memo) for _, i in todo) + 1):
            step = [(b, i) for b, i in todo if _t_depth(i, memo) == d]
            pairs = []
            for b, i in step:
                x, y = b._operands(i)
                pairs.append((b.cache[x], b.cache[x] if x == y else b.cache[y]))
            cc = step[0][0].cc
            many = getattr(cc, "RescaleMany", None)
            prods = _mult_many(cc, pairs)
            if many is not None and len(step) > 1:
                values = many([b._unsettled(i, p) for (b, i), p in zip(step, prods)])
                for (b, i), v in zip(step, values):
                    b.cache[i] = v
            else:
                for (b, i), p in zip(step, prods):
                    b._finish(i, p)


def _ps_split(c, n: int, k: int):
    """p = rem + T_k quot for sum_{i<=n} c_i T_i, from T_k T_j =
    (T_{k+j} + T_{k-j}) / 2 (coefficients scalars or arrays)."""
    quot = [c[k]] + [2.0 * c[k + j] for j in range(1, n - k + 1)]
    rem = list(c[:k])
    for i in range(k + 1, n + 1):
        rem[2 * k - i] = rem[2 * k - i] - c[i]
    return rem, quot


class _PsNode:
    """A node of the Paterson-Stockmeyer recursion: a leaf series (degree
    below the baby size) or the split p = rem + T_k quot."""

    def __init__(self, c: list, m: int):
        n = len(c) - 1
        self.value = None
        if n < m:
            self.c, self.k, self.rem, self.quot, self.height = c, 0, None, None, 0
        else:
            self.k = _giant_split(n, m)
            rem, quot = _ps_split(c, n, self.k)
            self.c, self.rem, self.quot = None, _PsNode(rem, m), _PsNode(quot, m)
            self.height = 1 + max(self.rem.height, self.quot.height)

    def nodes(self):
        yield self
        if self.c is None:
            yield from self.rem.nodes()
            yield from self.quot.nodes()


def chebyshev_ps_many(cc, jobs):
    """sum_i coeffs[i] T_i(u) by Paterson-Stockmeyer
    (src/fhemamba/ckks_probes.py:108-155) for every job (u, coeffs, floor,
    const_ct) of independent inputs, in lockstep: the basis powers of one
    depth, then the giant-step products of one tree height, of every job
    are multiplied together (_mult_many).  Each job's result is the one
    chebyshev_ps gives.  `const_ct(value)` supplies a constant ciphertext
    when no term of a series survives its coefficient floor."""
    results = [None] * len(jobs)
    trees = []
    for j, (u, coeffs, floor, const_ct) in enumerate(jobs):
        def constant(value: float, const_ct=const_ct):
            if const_ct is None:
                raise ValueError("Chebyshev series has no term above the coefficient floor")
            return const_ct(value)

        degree = len(coeffs) - 1
        if degree < 1:
            results[j] = constant(coeffs[0] if len(coeffs) else 0.0)
            continue
        root = _PsNode(list(coeffs), cheb_baby_size(degree))
        trees.append((j, ChebBasis(cc, u), root, floor, constant))
    requests = []
    for _, basis, root, floor, _ in trees:
        need = set()
        for node in root.nodes():
            if node.c is None:
                need.add(node.k)
            else:
                need.update(i for i in range(1, len(node.c)) if abs(node.c[i]) >= floor)
        requests.append((basis, need))
    ChebBasis.build_many(requests)
    # with EvalLinearWSum a leaf's sum of c_i T_i is one weighted sum at the
    # deepest T_i level instead of products aligned pairwise (same value)
    wsum = getattr(cc, "EvalLinearWSum", None)
    splits = []
    for _, basis, root, floor, constant in trees:
        for node in root.nodes():
            if node.c is None:
                splits.append((basis, node))
                continue
            c = node.c
            idx = [i for i in range(1, len(c)) if abs(c[i]) >= floor]
            acc = None
            if idx and wsum is not None:
                acc = wsum([basis(i) for i in idx], [c[i] for i in idx])
            else:
                for i in idx:
                    term = cc.EvalMult(basis(i), c[i])
                    acc = term if acc is None else cc.EvalAdd(acc, term)
            if acc is None:
                acc = constant(c[0])
            elif abs(c[0]) >= floor:
                acc = cc.EvalAdd(acc, c[0])
            node.value = acc
    for h in sorted({node.height for _, node in splits}):
        step = [(basis, node) for basis, node in splits if node.height == h]
        giants = _mult_many(cc, [(basis(node.k), node.quot.value) for basis, node in step])
        for (_, node), giant in zip(step, giants):
            node.value = cc.EvalAdd(node.rem.value, giant)
    for j, _, root, _, _ in trees:
        results[j] = root.value
    return results


def chebyshev_ps(cc, u, coeffs: Sequence[float], floor: float = CHEB_COEFF_FLOOR,
                 const_ct=None):
    """sum_i coeffs[i] T_i(u) by Paterson-Stockmeyer
    (src/fhemamba/ckks_probes.py:108-155).  `const_ct(value)` supplies a
    constant ciphertext when no term survives the coefficient floor."""
    return chebyshev_ps_many(cc, [(u, coeffs, floor, const_ct)])[0]


def chebyshev_ps_rows(basis: ChebBasis, rows, baby: int, mul, add, const):
    """sum_i rows[i] (.) T_i(u) with one coefficient per slot (rows[i] a
    vector): the vector-coefficient Paterson-Stockmeyer evaluation of
    native/fideslib_stage0/include/stage1_joint_gates.hpp:68-125 (same
    split as chebyshev_ps, baby-step size `baby` so that series of one input
    share the basis).  mul(ct, row, key) is a plaintext product, add(ct, row)
    a plaintext addition and const(row) a ciphertext holding row; `key`
    names the row's place in the recursion (a plaintext cache key).  Only
    all-zero rows are skipped: no coefficient threshold."""
    cc = basis.cc

    def evaluate(c: list, path: str):
        n = len(c) - 1
        if n < baby:
            acc = None
            for i in range(1, n + 1):
                if not np.any(c[i]):
                    continue
                term = mul(basis(i), c[i], (path, i))
                acc = term if acc is None else cc.EvalAdd(acc, term)
            if acc is None:
                return const(c[0])
            return add(acc, c[0]) if np.any(c[0]) else acc
        k = _giant_split(n, baby)
        rem, quot = _ps_split(c, n, k)
        giant = cc.EvalMult(basis(k), evaluate(quot, path + "q"))
        return cc.EvalAdd(evaluate(rem, path + "r"), giant)

    return evaluate([np.asarray(r, dtype=np.float64) for r in rows], "")


class CkksPrimitives:
    """Elementary encrypted helpers over an OpenFHE-shaped context."""

    def __init__(self, cc, keys, *, batch: int,
                 coefficient_floor: float = CHEB_COEFF_FLOOR) -> None:
        self.cc = cc
        self.keys = keys
        self.batch = batch
        self.coefficient_floor = coefficient_floor
        # Constants are produced from an encrypted all-ones vector.
        self.ones_ct = self.encrypt(np.ones(batch))

    def encrypt(self, values: np.ndarray, fill: float = 0.0):
        """Encrypt `values`, padding the unused slots with `fill`."""
        slots = np.full(self.batch, float(fill))
        slots[: len(values)] = values
        pt = self.cc.MakeCKKSPackedPlaintext([float(x) for x in slots])
        return self.cc.Encrypt(self.keys.publicKey, pt)

    def decrypt(self, ct, n: int | None = None) -> np.ndarray:
        pt = self.cc.Decrypt(ct, self.keys.secretKey)
        pt.SetLength(self.batch)
        return np.asarray(pt.GetRealPackedValue(), dtype=np.float64)[:n]

    def mask_mult(self, ct, mask: np.ndarray):
        return self.cc.EvalMult(ct, self.cc.MakeCKKSPackedPlaintext([float(x) for x in mask]))

    def const_ct(self, value: float):
        return self.cc.EvalMult(self.ones_ct, float(value))

    def affine_ct(self, ct, a: float, b: float):
        """a * ct + b (one level)."""
        return self.cc.EvalAdd(self.cc.EvalMult(ct, float(a)), float(b))

    def eval_chebyshev(self, u, coeffs: Sequence[float]):
        """sum_i coeffs[i] T_i(u) by Paterson-Stockmeyer."""
        return chebyshev_ps(self.cc, u, coeffs, self.coefficient_floor, self.const_ct)

    def newton_refine(self, y, v_neg_half, iterations: int):
        """Newton steps for 1/sqrt(v): y <- 1.5 y + (-v/2) * y * y^2."""
        cc = self.cc
        for _ in range(iterations):
            y_sq = cc.EvalMult(y, y)
            vy = cc.EvalMult(v_neg_half, y)
            cube = cc.EvalMult(vy, y_sq)
            y = cc.EvalAdd(cc.EvalMult(y, 1.5), cube)
        return y


def build_toy_context(*, ring_dimension, batch, depth, scale_bits, first_mod_bits,
                      rotations=(), backend=None, seed=None, secret_dist=None):
    """CKKS context with TOY security for probes: uniform-ternary secret
    (unless `secret_dist` names another SecretKeyDist member), FLEXIBLEAUTO,
    HYBRID, explicit ring dimension and batch; keys for multiplication and
    the given rotations.  `backend` is any module with the OpenFHE names
    (default: fhemamba_amd.ckks)."""
    if backend is None:
        from . import ckks as backend
    params = backend.CCParamsCKKSRNS()
    params.SetSecretKeyDist(getattr(backend.SecretKeyDist, secret_dist or "UNIFORM_TERNARY"))
    params.SetSecurityLevel(backend.SecurityLevel.HEStd_NotSet)
    params.SetRingDim(ring_dimension)
    params.SetScalingTechnique(backend.ScalingTechnique.FLEXIBLEAUTO)
    params.SetFirstModSize(first_mod_bits)
    params.SetScalingModSize(scale_bits)
    params.SetKeySwitchTechnique(backend.KeySwitchTechnique.HYBRID)
    params.SetMultiplicativeDepth(depth)
    params.SetBatchSize(batch)
    cc = backend.GenCryptoContext(params) if seed is None else \
        backend.GenCryptoContext(params, seed=seed)
    features = backend.PKESchemeFeature
    for f in (features.PKE, features.KEYSWITCH, features.LEVELEDSHE, features.ADVANCEDSHE,
              features.FHE):
        cc.Enable(f)
    keys = cc.KeyGen()
    cc.EvalMultKeyGen(keys.secretKey)
    if rotations:
        cc.EvalRotateKeyGen(keys.secretKey, list(rotations))
    return cc, keys
