"""Encrypted Mamba-2 SSM layer step: state update and readout.

Semantics (per head h, channel p, state index n):
    decay_h   = exp(dt_h * A_h)
    h'[h,p,n] = decay_h * h[h,p,n] + (dt_h * x[h,p]) * B[n]
    y[h,p]    = sum_n h'[h,p,n] * C[n] + D_h * x[h,p]
following src/fhemamba/tensor_ops.py:59-120 (ssm_readout,
ssm_update_readout: decay, rank-one write of value * dt with key B, readout
against C) and src/fhemamba/ops.py:76-80 (decay = exp(dt * A)); D * x is
the skip term of the Mamba-2 block.

Packing follows native/fideslib_stage0/src/stage1_mamba2_decode_fideslib.cpp
:23-27: a state ciphertext holds heads_per_ct whole heads at slot
n * group_block + h_local * headdim + p (group_block = heads_per_ct *
headdim); the readout's sum over n is a rotate-sum by group_block * 2^k
(:4047-4052), after which group g's outputs are masked to the first block
and rotated to offset g * group_block of one compact y (h * headdim + p).
The per-group inputs x, dt (and the per-head constants A, D) arrive
"expanded" to that layout, B and C replicated over (h_local, p), as the
reference's projection and expand stages deliver them.

The decay uses range reduction, exp(t) = exp(t / 2^k)^(2^k): a Chebyshev
interpolant of exp on [-amax / 2^k, 0] evaluated by Paterson-Stockmeyer
(ckks_probes.CkksPrimitives.eval_chebyshev), then k squarings.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from .ckks_probes import CkksPrimitives, cheb_ps_depth


@dataclass(frozen=True)
class SSMShape:
    nheads: int = 24
    headdim: int = 64
    d_state: int = 128
    slots: int = 32768

    def __post_init__(self):
        per = self.headdim * self.d_state
        if self.slots % per or self.nheads % (self.slots // per):
            raise ValueError("slots must hold whole heads and the heads whole ciphertexts")
        if self.d_state & (self.d_state - 1):
            raise ValueError("d_state must be a power of two (rotate-sum readout)")

    @property
    def heads_per_ct(self) -> int:
        return self.slots // (self.headdim * self.d_state)

    @property
    def group_block(self) -> int:
        return self.heads_per_ct * self.headdim

    @property
    def groups(self) -> int:
        return self.nheads // self.heads_per_ct

    @property
    def d_inner(self) -> int:
        return self.nheads * self.headdim


# ----------------------------------------------------------------- packing
def pack_state(h: np.ndarray, shape: SSMShape) -> list[np.ndarray]:
    """h [nheads][headdim][d_state] -> one slot vector per group."""
    hp, gb = shape.heads_per_ct, shape.group_block
    out = []
    for g in range(shape.groups):
        blk = h[g * hp:(g + 1) * hp]                     # [hp][p][n]
        out.append(np.ascontiguousarray(blk.transpose(2, 0, 1)).reshape(shape.d_state * gb))
    return out


def unpack_state(vecs: Sequence[np.ndarray], shape: SSMShape) -> np.ndarray:
    hp = shape.heads_per_ct
    h = np.empty((shape.nheads, shape.headdim, shape.d_state))
    for g, v in enumerate(vecs):
        blk = np.asarray(v)[: shape.slots].reshape(shape.d_state, hp, shape.headdim)
        h[g * hp:(g + 1) * hp] = blk.transpose(1, 2, 0)
    return h


def expand_channels(x: np.ndarray, shape: SSMShape) -> list[np.ndarray]:
    """x [nheads][headdim] -> per group, x[h][p] at every n."""
    hp = shape.heads_per_ct
    return [np.tile(x[g * hp:(g + 1) * hp].reshape(-1), shape.d_state)
            for g in range(shape.groups)]


def expand_heads(v: np.ndarray, shape: SSMShape) -> list[np.ndarray]:
    """v [nheads] -> per group, v[h] at every (n, p) of head h."""
    return expand_channels(np.repeat(np.asarray(v, float)[:, None], shape.headdim, 1), shape)


def expand_states(b: np.ndarray, shape: SSMShape) -> np.ndarray:
    """b [d_state] -> b[n] at every (h_local, p) of block n."""
    return np.repeat(np.asarray(b, float), shape.group_block)


def ssm_step_reference(h, x, dt, A, B, C, D):
    """float64 reference: returns (h', y)."""
    decay = np.exp(dt * A)
    h2 = decay[:, None, None] * h + (dt[:, None] * x)[:, :, None] * B[None, None, :]
    y = np.einsum("hpn,n->hp", h2, C) + D[:, None] * x
    return h2, y


# ----------------------------------------------------------------- decay
@dataclass(frozen=True)
class DecayPolynomial:
    """exp(t) for t in [-amax, 0] as exp(t / 2^k)^(2^k): the Chebyshev
    interpolant (degree `degree`) of exp on [-amax / 2^k, 0], in the
    variable u = 2 t / amax + 1 in [-1, 1]."""
    amax: float
    squarings: int = 5
    degree: int = 13

    @property
    def coeffs(self) -> list[float]:
        w = self.amax / 2 ** self.squarings
        f = lambda u: np.exp((u - 1.0) * w / 2.0)  # noqa: E731
        return [float(c) for c in np.polynomial.chebyshev.chebinterpolate(f, self.degree)]

    def u_scale(self) -> float:
        """u = dt * A * u_scale + 1."""
        return 2.0 / self.amax

    def plain(self, t: np.ndarray) -> np.ndarray:
        u = np.asarray(t) * self.u_scale() + 1.0
        e = np.polynomial.chebyshev.chebval(u, self.coeffs)
        for _ in range(self.squarings):
            e = e * e
        return e

    def depth(self) -> int:
        return 1 + cheb_ps_depth(self.degree) + self.squarings


# ----------------------------------------------------------------- encrypted step
class EncryptedSSMStep:
    """One SSM layer step on encrypted inputs over an OpenFHE-shaped context.

    Plaintext weights: A, D [nheads].  Encrypted inputs per step: the state
    groups, x expanded per group, dt expanded per group, B and C replicated,
    and x in compact layout (for D * x).  Needs rotation keys for
    group_block * 2^k (k < log2 d_state) and -group_block * g (g < groups);
    rotation_indices() lists them."""

    def __init__(self, cc, keys, shape: SSMShape, A: np.ndarray, D: np.ndarray,
                 decay: DecayPolynomial):
        self.cc, self.keys, self.shape, self.decay = cc, keys, shape, decay
        self.A, self.D = np.asarray(A, float), np.asarray(D, float)
        s = shape
        self.he = CkksPrimitives(cc, keys, batch=s.slots)
        scale = decay.u_scale()
        self._a_pt = [cc.MakeCKKSPackedPlaintext(list(v)) for v in
                      expand_heads(self.A * scale, s)]
        mask = np.zeros(s.slots)
        mask[: s.group_block] = 1.0
        self._mask_pt = cc.MakeCKKSPackedPlaintext(list(mask))
        d_compact = np.zeros(s.slots)
        d_compact[: s.d_inner] = np.repeat(self.D, s.headdim)
        self._d_pt = cc.MakeCKKSPackedPlaintext(list(d_compact))
        self._coeffs = decay.coeffs

    def rotation_indices(self) -> list[int]:
        s = self.shape
        sums = [s.group_block << k for k in range(int(math.log2(s.d_state)))]
        places = [-s.group_block * g for g in range(1, s.groups)]
        return sums + places

    def _rotate_all(self, cts: list, index: int) -> list:
        if hasattr(self.cc, "EvalRotateMany"):
            return self.cc.EvalRotateMany(cts, index)
        return [self.cc.EvalRotate(c, index) for c in cts]

    def __call__(self, state: list, x_groups: list, dt_groups: list, b_ct, c_ct, x_compact):
        cc, s = self.cc, self.shape
        new_state, reads = [], []
        for g in range(s.groups):
            # decay = exp(dt * A): u = dt * A * scale + 1, PS Chebyshev, squarings
            u = cc.EvalAdd(cc.EvalMult(dt_groups[g], self._a_pt[g]), 1.0)
            e = self.he.eval_chebyshev(u, self._coeffs)
            for _ in range(self.decay.squarings):
                e = cc.EvalSquare(e)
            write = cc.EvalMult(cc.EvalMult(x_groups[g], dt_groups[g]), b_ct)
            h2 = cc.EvalAdd(cc.EvalMult(e, state[g]), write)
            new_state.append(h2)
            reads.append(cc.EvalMult(h2, c_ct))
        # sum over n: rotate-sum by group_block * 2^k on all groups at once
        for k in range(int(math.log2(s.d_state))):
            rot = self._rotate_all(reads, s.group_block << k)
            reads = [cc.EvalAdd(r, t) for r, t in zip(reads, rot)]
        # group g's block 0 -> offset g * group_block of one compact y
        masked = [cc.EvalMult(r, self._mask_pt) for r in reads]
        placed = [masked[0]]
        if s.groups > 1:
            placed += self._rotate_many_indices(masked[1:], [-s.group_block * g
                                                             for g in range(1, s.groups)])
        y = placed[0]
        for t in placed[1:]:
            y = cc.EvalAdd(y, t)
        y = cc.EvalAdd(y, cc.EvalMult(x_compact, self._d_pt))
        return new_state, y

    def _rotate_many_indices(self, cts: list, indices: list) -> list:
        if hasattr(self.cc, "EvalRotateMany"):
            return self.cc.EvalRotateMany(cts, indices)
        return [self.cc.EvalRotate(c, i) for c, i in zip(cts, indices)]

    def depth(self) -> int:
        """Levels consumed from the inputs to y."""
        return max(self.decay.depth(), 2) + 1 + 1 + 1
