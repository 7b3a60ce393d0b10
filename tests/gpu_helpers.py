"""Shared helpers for the GPU parity tests (inputs, contexts, oracle pairs)."""
import numpy as np

import oracle as O


def residues(rng, mods, shape_prefix, n):
    """Uniform residues [*, len(mods), n], limb j uniform in [0, mods[j])."""
    out = np.empty((*shape_prefix, len(mods), n), dtype=np.uint64)
    for j, q in enumerate(mods):
        out[..., j, :] = rng.integers(0, q, (*shape_prefix, n), dtype=np.uint64)
    return out


def edge_patterns(mods, n):
    """The four probe patterns of experiments/ntt_warp_tail/probe.cu:41-55:
    zero, q-1, alternating 0/q-1 and mixed."""
    pats = []
    for kind in range(4):
        a = np.zeros((len(mods), n), dtype=np.uint64)
        for j, q in enumerate(mods):
            if kind == 1:
                a[j] = q - 1
            elif kind == 2:
                a[j, 1::2] = q - 1
            elif kind == 3:
                a[j] = (np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15 % q)) % np.uint64(q)
        pats.append(a)
    return np.stack(pats)


def scheme(log_n, depth, scale_bits, first_bits, dnum):
    q, p = O.gen_moduli(log_n, depth, scale_bits, first_bits, dnum)
    return q, p
