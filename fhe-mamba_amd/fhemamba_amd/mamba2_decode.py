"""Encrypted Mamba-2 decode from a chain payload: a drop-in for the token
and layer loops of native/fideslib_stage0/src/stage1_mamba2_decode_fideslib.cpp
(run_layer :3634-4232, token loop :4287, layer loop :4388) over this
package's CKKS interface on the GPU.

Per layer (semantics of fhemamba_amd.mamba2_payload.layer_step, the payload's
polynomial circuit), all ciphertexts of `slots` = N/2 slots:
  * block norm: hidden^2 summed over every slot by rotate-adds (zero padding
    makes the total land in every slot), v = total / d_model + eps,
    inverse square root by the payload's Chebyshev guess + Newton steps;
    normed = hidden * inv;
  * in_proj by the replicated baby-step giant-step matvec (block_norm_w
    folded into the weights); proj holds z | xBC | dt at slots
    [0, d_inner) | [d_inner, d_inner + conv_dim) | the rest;
  * conv: the FIFO keeps the last conv_kernel - 1 proj ciphertexts; taps
    and bias are plaintext vectors on the xBC slots (the reference's "taps
    multiply xBC slots of the raw proj ciphertexts", :3741-3760); SiLU by
    the payload's Chebyshev series;
  * gates: SiLU(z); dt = (Chebyshev sqrt-softplus)^2 on dt + dt_bias;
    decay = exp(dt A) by Chebyshev and squarings, times the head mask;
    with a joint gate (JointGateSpec) instead: per-head affine map of
    dt + dt_bias onto [-1, 1], the two per-head Chebyshev series p and q by
    a vector-coefficient Paterson-Stockmeyer over one shared basis
    (:3781-3830), write = p^2 q^2 in place of dt and decay = 1 - p^2;
  * SSM in the reference's packing (:23-27): state group g holds heads
    heads_per_ct g ... at slot n * group_block + h_local * head_dim + p;
    x, dt and decay are expanded to it (a rotation, a mask, a rotate-sum
    over n), B and C replicated (a one-level diagonal scatter of B[n] to
    n * group_block, then a rotate-sum over the block); h' = decay h +
    (dt x) B; readout h' C rotate-summed over n, masked and placed; + D x;
  * gated norm of y * SiLU(z) with the payload's squared-guess Newton
    inverse square root; out_proj (gated_norm_w folded); residual add.
The final hidden goes through RMSNorm with final_norm_w.

Refresh: before each phase every input ciphertext whose level plus the
phase's level need would pass the ceiling is scaled into [-1, 1] by a
public bound, bootstrapped (two passes for the carried and other
precision-critical values, one for the rest; EncryptedMamba2Decoder's
constructor lists them) and scaled back, as the reference's
maybe_bootstrap checkpoints do (:2127-2297).  Bounds are public calibration
maxima (payload `carried_bounds`, else the defaults below), never values
read from ciphertexts.
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field

import numpy as np

from .ckks_probes import (ChebBasis, affine, cheb_baby_size, cheb_ps_depth, chebyshev_ps_many,
                          chebyshev_ps_rows)
from .mamba2_payload import ChainPayload, JointGateSpec, LayerPayload, PolySpec
from .packed import PackedEvaluator, replicated_shape

# Refresh bounds by checkpoint where a payload carries no calibration maxima
# (with maxima: BOUND_MARGIN times the payload's value).
DEFAULT_BOUNDS = {"residual": 64.0, "variance": 64.0, "inv": 64.0, "proj_raw": 64.0,
                  "proj": 16.0, "conv": 16.0, "act": 16.0, "gate": 16.0, "dt": 16.0,
                  "decay": 1.0, "state": 64.0, "y": 64.0, "gated": 64.0,
                  "gated_variance": 64.0, "gated_inv": 64.0, "out_raw": 64.0,
                  "output": 64.0, "out_residual": 64.0, "out_variance": 64.0,
                  "out_inv": 64.0}
BOUND_MARGIN = 2.0


@dataclass
class LayerCtState:
    ssm: list | None = None            # state group ciphertexts (None: zero)
    fifo: list = field(default_factory=list)   # previous proj ciphertexts, oldest first


class EncryptedMamba2Decoder:
    def __init__(self, cc, keys, chain: ChainPayload, *, bootstrap_passes: int = 2,
                 transient_passes: int = 1, refresh_ceiling: int | None = None,
                 bounds: dict | None = None, log=None, s2c_first: bool = False,
                 level_budget=(4, 4)):
        first = chain.layers[0]
        self.chain, self.cc = chain, cc
        self.slots = cc.GetBatchSize()
        self.log = log or (lambda m: None)
        self.ev = PackedEvaluator(cc, keys, self.slots, bootstrap_passes=bootstrap_passes,
                                  refresh_ceiling=refresh_ceiling, log=self.log,
                                  s2c_first=s2c_first, level_budget=tuple(level_budget))
        # Refresh passes by site, the reference decoder's Meta-BTS rule
        # (should_use_meta_bts, stage1_mamba2_config.cpp:69-86, with
        # is_carried_checkpoint, stage1_mamba2_decode_fideslib.cpp:218-220):
        # two-pass refreshes (bootstrap_passes) for the carried lineages
        # (SSM state, conv-window entries refreshed out of the FIFO), the
        # gated norm's polynomial input, the residual of the last three
        # layers, the final output and every refresh inside a scheduled
        # normalization; one pass (transient_passes) for the other values,
        # the new projection among them (it enters the FIFO fresh).
        if transient_passes not in (1, 2):
            raise ValueError("transient bootstrap passes must be 1 or 2")
        self.critical_passes = bootstrap_passes
        self.transient_passes = min(transient_passes, bootstrap_passes)
        self._critical_residual = set(range(max(0, len(chain.layers) - 3), len(chain.layers)))
        self.bounds = [self._layer_bounds(lay, bounds) for lay in chain.layers]
        self.d, self.di, self.ns = first.d_model, first.d_inner, first.state_size
        self.nh, self.hd, self.kc = first.num_heads, first.head_dim, first.conv_kernel
        self.cd = first.conv_dim
        per = self.hd * self.ns
        # heads per state ciphertext: the largest power of two that divides
        # the head count and fits the slots (the state's rotate-sums walk
        # power-of-two block strides)
        hp = 1
        while self.nh % (2 * hp) == 0 and 2 * hp * per <= self.slots:
            hp *= 2
        if per > self.slots or self.slots % per or per & (per - 1):
            raise ValueError("slots must hold whole heads and the heads whole ciphertexts")
        self.hp = hp                                   # heads per state ciphertext
        self.gb = self.hp * self.hd                    # group block
        self.groups = self.nh // self.hp
        if first.proj_dim > self.slots or self.d > self.slots:
            raise ValueError("the projection does not fit one ciphertext")
        self.stats = dict(tokens=0, layers=0)

    # ------------------------------------------------------------ helpers
    def _vec(self, entries: dict) -> np.ndarray:
        v = np.zeros(self.slots)
        for start, values in entries.items():
            values = np.atleast_1d(np.asarray(values, dtype=np.float64))
            v[start:start + len(values)] = values
        return v

    def _support(self, start: int, size: int) -> np.ndarray:
        return self._vec({start: np.ones(size)})

    @staticmethod
    def _layer_bounds(lay: LayerPayload, override) -> dict:
        b = dict(DEFAULT_BOUNDS)
        for k, v in lay.bounds.items():
            b[k] = max(BOUND_MARGIN * float(v), 1e-12)
        if lay.joint is not None:
            # a joint gate's write and decay take the refresh bounds its
            # coefficients certify (the calibration "dt" is softplus's)
            w, d = lay.joint.bounds()
            b["dt"], b["decay"] = BOUND_MARGIN * w, BOUND_MARGIN * d
        b.update(override or {})
        return b

    def ready(self, ct, need: int, bound: float, support=None, critical: bool = False,
              passes: int | None = None):
        """Refresh ct (masked to `support`) if `need` more levels would pass
        the ceiling; `critical` refreshes take the two-pass count, `passes`
        overrides both."""
        if self.ev._level(ct) + need > self.ev.refresh_ceiling:
            if passes is None:
                passes = self.critical_passes if critical else self.transient_passes
            return self.ev.refresh(ct, bound, support if support is not None else self.slots,
                                   passes)
        return ct

    def ready_many(self, cts, need: int, bound: float, support=None, critical: bool = False):
        """ready() of each ciphertext of `cts` (one bound and support), the
        ones that need a refresh refreshed together."""
        ev = self.ev
        out = list(cts)
        idx = [i for i, ct in enumerate(out) if ev._level(ct) + need > ev.refresh_ceiling]
        if idx:
            fresh = ev.refresh_many([out[i] for i in idx], bound,
                                    support if support is not None else self.slots,
                                    self.critical_passes if critical else self.transient_passes)
            for i, ct in zip(idx, fresh):
                out[i] = ct
        return out

    def full_sum(self, ct):
        """Every slot gets the sum over all slots (rotate-adds)."""
        step = 1
        while step < self.slots:
            ct = self.ev.add(ct, self.ev.rotate(ct, step))
            step *= 2
        return ct

    def cheb(self, x, spec: PolySpec, support: np.ndarray, squarings_scale: int = 0):
        """Chebyshev series of `spec` on the supported slots (domain scaled
        by 2^squarings_scale for the range-reduced exp)."""
        return self.cheb_many([(x, spec, support, squarings_scale)])[0]

    def cheb_many(self, series):
        """cheb(x, spec, support, squarings_scale) of every entry of
        `series` (independent inputs), the series' products of one step
        relinearized together."""
        jobs = []
        for x, spec, support, squarings_scale in series:
            lo, hi = spec.lo * 2 ** squarings_scale, spec.hi * 2 ** squarings_scale
            u = self.ev.plain(x, support * (2.0 / (hi - lo)), True)
            u = self.ev.plain(u, support * (-(lo + hi) / (hi - lo)), False)
            jobs.append((u, [float(c) for c in spec.coeffs], 1e-14,
                         lambda v, u=u: self.ev.scale(u, 0.0)))
        return chebyshev_ps_many(self.cc, jobs)

    def cheb_need(self, spec: PolySpec) -> int:
        return 1 + cheb_ps_depth(len(spec.coeffs) - 1) + 1

    @staticmethod
    def joint_need(spec: JointGateSpec) -> int:
        """Levels from dt + dt_bias to write and decay: the affine map, the
        deeper series, p^2 and q^2, their product (decay's negating mask is
        no deeper)."""
        m = cheb_baby_size(max(spec.degree, 1))
        return 1 + max(cheb_ps_depth(len(c) - 1, m) for c in (spec.p, spec.q)) + 2

    def joint_gates(self, li: int, dtin, spec: JointGateSpec, d0: int):
        """(write, decay) of a joint gate for dt + dt_bias at slots
        [d0, d0 + nh): u = a_h (dt + dt_bias) + b_h maps each head's domain
        onto [-1, 1]; p and q share one Chebyshev basis of u."""
        ev = self.ev
        ab = [affine(lo, hi) for lo, hi in zip(spec.lo, spec.hi)]
        u = ev.plain(dtin, self._vec({d0: [a for a, _ in ab]}), True, key=("joint_a", li))
        u = ev.plain(u, self._vec({d0: [b for _, b in ab]}), False)
        basis = ChebBasis(self.cc, u)
        baby = cheb_baby_size(max(spec.degree, 1))

        def series(coeffs, name):
            rows = [self._vec({d0: r}) for r in coeffs]
            return chebyshev_ps_rows(
                basis, rows, baby,
                lambda ct, row, key: ev.plain(ct, row, True, key=("joint", li, name) + key),
                lambda ct, row: ev.plain(ct, row, False),
                lambda row: ev.plain(ev.scale(u, 0.0), row, False))

        p, q = series(spec.p, "p"), series(spec.q, "q")
        d = ev.mul(p, p)
        write = ev.mul(d, ev.mul(q, q))
        decay = ev.plain(ev.plain(d, self._vec({d0: -np.ones(self.nh)}), True,
                                  key=("joint_neg", d0)),
                         self._vec({d0: np.ones(self.nh)}), False)
        return write, decay

    def sched_inv_sqrt(self, v, spec, vbound: float, ibound: float):
        """Scheduled normalization (ScheduledInvSqrtSpec): u = v seed^2 in
        (0, 1], per stage f = a - b u, y <- y f, u <- u f^2, then the
        recomputed Newton step y (1.5 - 0.5 v y^2).  The schedule keeps u in
        (0, 1] and y below 1 / sqrt(v), so u refreshes at bound 1, y at the
        inverse's bound and f at the largest a."""
        ev, cc = self.ev, self.cc
        fbound = BOUND_MARGIN * max(a for a, _ in spec.coefficients)
        ubound = BOUND_MARGIN
        n = len(spec.coefficients)
        v = self.ready(v, 3, vbound, critical=True)
        u = ev.scale(v, spec.seed * spec.seed)
        y = None
        for i, (a, b) in enumerate(spec.coefficients):
            u = self.ready(u, 4, ubound, critical=True)
            f = cc.EvalAdd(ev.scale(u, -b), a)
            if y is None:
                y = ev.scale(f, spec.seed)
            else:
                y = ev.mul(self.ready(y, 1, ibound, critical=True),
                           self.ready(f, 1, fbound, critical=True))
            if i + 1 < n:
                f = self.ready(f, 2, fbound, critical=True)
                u = ev.mul(u, ev.mul(f, f))
        y = self.ready(y, 3, ibound, critical=True)
        v = self.ready(v, 2, vbound, critical=True)
        t = ev.mul(v, ev.mul(y, y))
        return ev.mul(y, cc.EvalAdd(ev.scale(t, -0.5), 1.5))

    def inv_sqrt(self, v, spec: PolySpec, vbound: float, ibound: float):
        """The payload's Newton inverse square root of v (v in every slot,
        so refreshes need no mask)."""
        if spec.kind == "scaled-goldschmidt-invsqrt-v1":
            return self.sched_inv_sqrt(v, spec, vbound, ibound)
        v = self.ready(v, self.cheb_need(spec) + 2, vbound)
        q = self.cheb(v, spec, np.ones(self.slots))
        if spec.kind == "poly-newton":
            y = self.ev.scale(q, 0.9)
        elif spec.kind == "sq-poly-newton":
            y = self.ev.scale(self.ev.mul(q, q), spec.damping)
        else:
            raise ValueError(f"inverse square root of kind {spec.kind}")
        vh = self.ev.scale(v, -0.5)
        for _ in range(spec.iterations):
            # y's refresh is followed by a Newton step, whose map has zero
            # derivative at the root: a relative error e there leaves
            # -1.5 e^2, so one pass serves whatever the secret (vh's error
            # would move the root and keeps the transient count)
            y = self.ready(y, 3, ibound, passes=1)
            vh = self.ready(vh, 3, vbound)
            t = self.ev.mul(vh, self.ev.mul(y, y))
            y = self.ev.mul(y, self.cc.EvalAdd(t, 1.5))
        return y

    def decay_policy(self, decay_level: int, state_level: int) -> bool:
        """Refresh the compact decay before its expansion when its groups
        (two levels deeper) would drag the carried state deeper than the
        state itself: h' = decay h + ... takes the deeper operand's level, so
        a deep decay makes all state groups refresh within a token or two
        (one bootstrap each), where one bootstrap of the decay keeps the
        state growing a level per token."""
        return decay_level + 2 > state_level

    def rms_scale(self, x, width: int, eps: float, spec: PolySpec, xbound: float,
                  vbound: float, ibound: float):
        """inv_sqrt(mean(x^2) + eps) of the first `width` slots, in every slot
        (a broadcast scalar: it commutes with a following matvec)."""
        x = self.ready(x, 3, xbound, self._support(0, width))
        tot = self.full_sum(self.ev.mul(x, x))
        v = self.cc.EvalAdd(self.ev.scale(tot, 1.0 / width), float(eps))
        return self.inv_sqrt(v, spec, vbound, ibound)

    def times_scale(self, x, inv, bound: float, support, ibound: float):
        x = self.ready(x, 1, bound, support)
        inv = self.ready(inv, 1, ibound)
        return self.ev.mul(x, inv)

    def expand_compact(self, ct, start: int):
        """Slots [start + g gb, start + (g+1) gb) of ct -> per group g, that
        block at every n (slot n gb + j)."""
        offs = [start + g * self.gb for g in range(self.groups)]
        rots = self.ev.rotate_hoisted(ct, offs)
        sup = self._support(0, self.gb)
        ms = [self.ev.plain(r, sup, True, key=("blk", self.gb)) for r in rots]
        # the groups' rotate-sums in lockstep, one batched key switch a step
        return self.ev.rotation_sum_many(ms, self.ns, -self.gb)

    def spread_heads(self, ct, start: int, gain: float = 1.0):
        """Per-head values at slots [start, start + nh) -> compact channel
        layout (gain times the value of head h at h hd + p)."""
        masks: dict = {}
        for h in range(self.nh):
            off = start + h - h * self.hd          # rot(x, off)[h hd] = x[start + h]
            masks.setdefault(off, np.zeros(self.slots))[h * self.hd] = gain
        lone = self.ev.transform(ct, masks, key=("spread", start, gain))
        return self.ev.rotation_sum(lone, self.hd, -1)

    def replicate_states(self, ct, start: int):
        """B[n] at slot start + n -> B[n] at every slot of block n (n gb + j)."""
        masks: dict = {}
        for n in range(self.ns):
            off = start + n - n * self.gb
            masks.setdefault(off, np.zeros(self.slots))[n * self.gb] = 1.0
        lone = self.ev.transform(ct, masks, key=("replicate", start))
        return self.ev.rotation_sum(lone, self.gb, -1)

    # ------------------------------------------------------------ layer
    def layer(self, li: int, hidden, st: LayerCtState):
        lay: LayerPayload = self.chain.layers[li]
        ev, cc, B = self.ev, self.cc, self.bounds[li]
        di, cd, ns, gb = self.di, self.cd, self.ns, self.gb
        t = lay.t
        # block norm: in_proj(hidden * inv) = in_proj(hidden) * inv, so the
        # matvec runs on the shallow residual (block_norm_w folded in); one
        # refresh of the residual serves the variance, the matvec and the
        # residual add
        res_critical = li in self._critical_residual
        hidden = self.ready(hidden, 4, B["residual"], self._support(0, self.d), res_critical)
        inv = self.rms_scale(hidden, self.d, lay.eps_block, lay.polys["rms_invsqrt"],
                             B["residual"], B["variance"], B["inv"])
        w_in = t("in_proj_w") * t("block_norm_w")[None, :]
        hin = hidden
        psup = self._support(0, lay.proj_dim)
        proj = self.times_scale(ev.linear(hin, w_in, ("in_proj", li)), inv, B["proj_raw"],
                                psup, B["inv"])
        # one refresh serves every consumer of proj (conv, gate, dt, FIFO)
        need = max(2, self.cheb_need(lay.polys["gate_silu"]),
                   self.cheb_need(lay.polys["dt_softplus"]) + 2 if lay.joint is None
                   else self.joint_need(lay.joint))
        proj = self.ready(proj, need, B["proj"], psup)
        # conv over the FIFO of raw proj ciphertexts (taps on the xBC slots)
        window = list(st.fifo) + [proj]
        xs = self._support(di, cd)
        pad = self.kc - len(window)
        conv = None
        for k, ct in enumerate(window):
            ct = self.ready(ct, 2, B["proj"], psup, critical=True)
            term = ev.plain(ct, self._vec({di: t("conv_w")[:, pad + k]}), True)
            conv = term if conv is None else ev.add(conv, term)
        conv = ev.plain(conv, self._vec({di: t("conv_b")}), False)
        conv = self.ready(conv, self.cheb_need(lay.polys["conv_silu"]), B["conv"], xs)
        # SiLU of the conv output, and the gates SiLU(z) and sqrt-softplus of
        # dt + dt_bias: independent series, evaluated in lockstep
        zs = self._support(0, di)
        d0 = di + cd
        ds = self._support(d0, self.nh)
        sp = lay.polys["dt_softplus"]
        dtin = ev.plain(proj, self._vec({d0: t("dt_bias")}), False)
        dec = lay.polys["decay_exp"]
        series = [(conv, lay.polys["conv_silu"], xs, 0), (proj, lay.polys["gate_silu"], zs, 0)]
        if lay.joint is None:
            series.append((dtin, sp, ds, 0))
        values = self.cheb_many(series)
        act = ev.plain(values[0], xs, True, key=("xbc", di, cd))
        gate = ev.plain(values[1], zs, True, key=("z", di))
        if lay.joint is None:
            q = values[2]
            dt = ev.plain(ev.mul(q, q), ds, True, key=("dt", d0))
            need_dt = self.cheb_need(dec) + dec.squarings + 6
        else:
            dt, decay = self.joint_gates(li, dtin, lay.joint, d0)
            need_dt = 6
        A = -np.exp(t("a_log"))
        # act (xBC slots) and dt (dt slots) occupy disjoint slots of the proj
        # layout: when either needs a refresh both go through one bootstrap,
        # dt first scaled by a power of two (exact, no level) into act's
        # range; every consumer below masks, and dt's masks carry 1 / f
        need_act = 7
        f = 1
        if max(ev._level(act) + need_act, ev._level(dt) + need_dt) > ev.refresh_ceiling:
            f = 1 << max(0, math.ceil(math.log2(B["act"] / B["dt"])))
            comb = ev.add(act, cc.MultByInteger(dt, f) if f > 1 else dt)
            comb = ev.refresh(comb, max(B["act"], B["dt"] * f), xs + ds, self.transient_passes)
            act = dt = comb
        if lay.joint is None:
            e = self.cheb(ev.plain(dt, self._vec({d0: A / f}), True), dec, ds, dec.squarings)
            for _ in range(dec.squarings):
                e = self.ev.mul(e, e)
            hm = dec.head_mask if dec.head_mask is not None else np.ones(self.nh)
            decay = ev.plain(e, self._vec({d0: hm}), True)
        # expansions into the state packing
        # compact values refreshed with room for the expansions and the
        # state update, so the expanded ciphertexts need no refresh
        act = self.ready(act, need_act, B["act"], xs)
        x_groups = self.expand_compact(act, di)
        b_rep = self.replicate_states(act, di + di)
        c_rep = self.replicate_states(act, di + di + ns)
        if f > 1:
            dt_c = self.spread_heads(dt, d0, 1.0 / f)
        else:
            dt_c = self.spread_heads(self.ready(dt, 6, B["dt"], ds), d0)
        dt_groups = self.expand_compact(dt_c, 0)
        decay = self.ready(decay, 5, B["decay"], ds)
        if st.ssm is not None and self.decay_policy(ev._level(decay), ev._level(st.ssm[0])):
            # a transient value (the carried checkpoint is the state)
            decay = self.ev.refresh(decay, B["decay"], ds, self.transient_passes)
        decay_groups = self.expand_compact(self.spread_heads(decay, d0), 0)
        # state update and readout; the groups' state refreshes (they reach
        # the ceiling together) go through one multi-ciphertext bootstrap
        xs_g = self.ready_many(x_groups, 4, B["act"])
        ds_g = self.ready_many(dt_groups, 4, B["dt"])
        br = self.ready(b_rep, 3, B["act"])
        writes = [ev.mul(ev.mul(xg, dg), br) for xg, dg in zip(xs_g, ds_g)]
        if st.ssm is not None:
            es_g = self.ready_many(decay_groups, 2, B["decay"])
            hs_g = self.ready_many(st.ssm, 2, B["state"], critical=True)
            h2s = [ev.add(ev.mul(eg, hg), w) for eg, hg, w in zip(es_g, hs_g, writes)]
        else:
            h2s = writes
        new_ssm = self.ready_many(h2s, 3, B["state"], critical=True)
        cr = self.ready(c_rep, 3, B["act"])
        reads = [ev.mul(h2, cr) for h2 in new_ssm]
        k = gb
        while k < self.slots:
            ev._ensure_keys([k])
            ev.stats["rotations"] += len(reads)
            rot = self.cc.EvalRotateMany(reads, k) if hasattr(self.cc, "EvalRotateMany") \
                else [self.cc.EvalRotate(r, k) for r in reads]
            reads = [ev.add(a, b) for a, b in zip(reads, rot)]
            k *= 2
        y = None
        for g, r in enumerate(reads):
            m = ev.plain(r, self._support(0, gb), True, key=("blk", gb))
            m = ev.rotate(m, -g * gb)
            y = m if y is None else ev.add(y, m)
        xc = ev.rotate(act, di)                                   # x at [0, di)
        skip = ev.plain(xc, self._vec({0: np.repeat(t("d_skip"), self.hd)}), True)
        y = ev.add(y, skip)
        # gated norm, out_proj, residual
        y = self.ready(y, 2, B["y"], zs)
        gate = self.ready(gate, 2, B["gate"], zs)
        gated = ev.mul(y, gate)
        # gated norm: out_proj(gated * inv2) = out_proj(gated) * inv2 (one
        # refresh of gated serves the variance and the matvec)
        gated = self.ready(gated, 4, B["gated"], zs, critical=True)
        inv2 = self.rms_scale(gated, di, lay.eps_gated, lay.polys["gated_rms_invsqrt"],
                              B["gated"], B["gated_variance"], B["gated_inv"])
        w_out = t("out_proj_w") * t("gated_norm_w")[None, :]
        # the carried state deepens gated a level a token: aligned to the
        # deepest level it can have here, out_proj's diagonals are encoded
        # once instead of every token
        gin = ev.at_level(gated, ev.refresh_ceiling - 4)
        dsup = self._support(0, self.d)
        out = self.times_scale(ev.linear(gin, w_out, ("out_proj", li)), inv2, B["out_raw"],
                               dsup, B["gated_inv"])
        hidden = self.ready(hidden, 1, B["residual"], dsup, res_critical)
        new_hidden = ev.add(hidden, out)
        fifo = (list(st.fifo) + [proj])[-(self.kc - 1):] if self.kc > 1 else []
        self.stats["layers"] += 1
        return new_hidden, LayerCtState(new_ssm, fifo)

    # ------------------------------------------------------------ token
    def initial_states(self) -> list:
        return [LayerCtState() for _ in self.chain.layers]

    def step(self, embedding, states: list):
        """One token: encrypt the embedding (client side), run every layer,
        final RMSNorm; returns (final ciphertext, new states)."""
        return self.step_ct(self.ev.encrypt(np.asarray(embedding, dtype=np.float64)), states)

    def step_ct(self, h, states: list):
        """One token from an encrypted embedding (a server that holds no
        secret key)."""
        new_states = []
        for li, st in enumerate(states):
            t0 = time.perf_counter()
            h, ns_ = self.layer(li, h, st)
            new_states.append(ns_)
            self.log(f"layer {li}: {time.perf_counter() - t0:.3f}s level {h.GetLevel()} "
                     f"bootstraps {self.ev.stats['bootstraps']}")
        last = self.chain.layers[-1]
        B = self.bounds[-1]
        h = self.ready(h, 3, B["out_residual"], self._support(0, self.d), critical=True)
        inv = self.rms_scale(h, self.d, self.chain.final_norm_eps, self.chain.final_invsqrt(),
                             B["out_residual"], B["out_variance"], B["out_inv"])
        final = self.ev.plain(h, self._vec({0: self.chain.final_norm_w}), True)
        final = self.times_scale(final, inv, B["out_residual"] * float(
            np.max(np.abs(self.chain.final_norm_w))), self._support(0, self.d), B["out_inv"])
        self.stats["tokens"] += 1
        return final, new_states

    def decrypt(self, ct) -> np.ndarray:
        return self.ev.decrypt(ct, self.d)


def expected_rotation_count(lay: LayerPayload, slots: int) -> dict:
    """Replicated shapes of the two projections (plaintext count per layer)."""
    s_in = replicated_shape(lay.proj_dim, lay.d_model, slots)
    s_out = replicated_shape(lay.d_model, lay.d_inner, slots)
    return {"in_proj_masks": s_in.per_replica, "out_proj_masks": s_out.per_replica}


def token_loop(dec: EncryptedMamba2Decoder, chain: ChainPayload, n_tok: int, ar=None,
               sync=lambda: None, log=print) -> dict:
    """Decode n_tok tokens with carried state: the payload's test embeddings,
    or with `ar` (AutoregressiveAssets) the client-in-loop greedy protocol;
    per token the seconds, the errors of the decrypted final hidden against
    the polynomial and exact references, the client's selections and the
    token's window on the monotonic clock (nanoseconds, the clock kernel
    traces are stamped with on this platform, so a trace can be split by
    token)."""
    states = dec.initial_states()
    out = dict(seconds=[], errors_poly=[], errors_exact=[], selected=[], client_seconds=0.0,
               bootstraps=[], decrypt_seconds=0.0, token0={}, windows_ns=[])
    selected = out["selected"]
    want_poly = ar.expected_poly_final if ar else chain.expected_poly_final
    want_exact = ar.expected_exact_final if ar else chain.expected_final

    def max_err(got, want) -> float:
        # A non-finite slot is a failed decrypt: the largest finite double,
        # never a silent zero (np.max propagates NaN, but keep it explicit).
        d = np.abs(got - want)
        return float(np.max(d)) if np.all(np.isfinite(d)) else 1.0e308

    for k in range(n_tok):
        sync()
        b0 = dec.ev.stats["bootstraps"]
        w0 = time.monotonic_ns()
        t = time.perf_counter()
        ct, states = dec.step(ar.input_for(k, selected) if ar else chain.input_embeddings[k],
                              states)
        sync()
        out["seconds"].append(time.perf_counter() - t)
        out["windows_ns"].append([w0, time.monotonic_ns()])
        out["bootstraps"].append(dec.ev.stats["bootstraps"] - b0)
        t = time.perf_counter()
        got = dec.decrypt(ct)
        out["decrypt_seconds"] += time.perf_counter() - t
        if ar is not None and k >= ar.prompt_tokens - 1:
            selected.append(ar.select(got))
            out["client_seconds"] += time.perf_counter() - t
        if k == 0:
            ref = want_poly[0] if want_poly is not None else want_exact[0]
            out["token0"] = {"decrypted": [float(v) for v in got[:8]],
                             "expected": [float(v) for v in ref[:8]],
                             "exact": [float(v) for v in want_exact[0][:8]]}
        if want_poly is not None:
            out["errors_poly"].append(max_err(got, want_poly[k]))
        out["errors_exact"].append(max_err(got, want_exact[k]))
        ep = out["errors_poly"][-1] if out["errors_poly"] else float("nan")
        log(f"token {k}: {out['seconds'][-1]:.2f}s error vs polynomial {ep:.2e} vs exact "
            f"{out['errors_exact'][-1]:.2e}"
            + (f" selected {selected[-1]}" if ar is not None and selected else ""))
    return out


# ----------------------------------------------------------------- command line
SECRET_KEY_DISTS = {"sparse-ternary": "SPARSE_TERNARY", "uniform-ternary": "UNIFORM_TERNARY"}


def default_transient_passes(secret_key_dist: str, bootstrap_passes: int) -> int:
    """Passes of the refreshes outside the precision-critical sites: one
    with a sparse-ternary secret (a single pass reaches ~2^-19 of the bound
    at N = 2^16; the 24-layer 130M decode stays within 3e-5 of the
    polynomial circuit), otherwise as many as the critical ones (a single
    pass with a uniform-ternary secret reaches ~2^-13 and the classical-128
    decode would exceed 1e-3)."""
    return 1 if secret_key_dist == "sparse-ternary" else bootstrap_passes


def _decode_setup(payload_dir, security, secret_key_dist, ring_dim, sizes=None):
    from .mamba2_payload import read_chain_payload
    from .packed import CLASSICAL128
    if security not in ("not-set", "128-classic"):
        raise ValueError("security must be not-set or 128-classic")
    classical = security == "128-classic"
    if secret_key_dist is None:
        secret_key_dist = "uniform-ternary" if classical else "sparse-ternary"
    if secret_key_dist not in SECRET_KEY_DISTS:
        raise ValueError(f"secret key distribution must be one of {sorted(SECRET_KEY_DISTS)}")
    if ring_dim and (classical or ring_dim < 4096 or ring_dim & (ring_dim - 1)):
        raise ValueError("ring_dim: a power of two >= 4096, and only with security not-set")
    chain = read_chain_payload(payload_dir)
    extra = dict(CLASSICAL128) if classical else ({"ring_dim": ring_dim} if ring_dim else {})
    # depth / scale_bits / first_mod_bits (the reference decoder's
    # --multiplicative-depth, --scaling-mod-size, --first-mod-size)
    extra.update(sizes or {})
    slots = extra.get("ring_dim", 65536) // 2
    return chain, classical, secret_key_dist, slots, extra


def _truncate(chain, layers: int) -> None:
    if layers:
        from .mamba2_payload import decode_tokens
        if not 1 <= layers <= chain.n_layers:
            raise ValueError("layers must be in 1..n_layers")
        chain.layers = chain.layers[:layers]
        chain.n_layers = layers
        chain.expected_final, _ = decode_tokens(chain, chain.input_embeddings, False)
        chain.expected_poly_final, _ = decode_tokens(chain, chain.input_embeddings, True)


def _build(slots, seed, secret_key_dist, extra):
    from . import ckks
    from .packed import build_context
    return build_context(slots, seed=seed, secret_dist=getattr(
        ckks.SecretKeyDist, SECRET_KEY_DISTS[secret_key_dist]), **extra)


def run_payload(payload_dir: str, *, tokens: int = 0, bootstrap_passes: int = 2,
                transient_passes: int | None = None, seed=None,
                secret_key_dist: str | None = None, security: str = "not-set",
                layers: int = 0, autoregressive: bool = False, s2c_first: bool = True,
                ring_dim: int = 0, sizes: dict | None = None, level_budget=(4, 4),
                log=print) -> dict:
    """Decode the payload's test embeddings in turn (carried state) and
    compare the decrypted outputs with its polynomial-circuit and exact
    references; returns the report.

    security "not-set": N=2^16, 32768 slots, depth 44, dnum 3, and a sparse
    ternary secret by default, as the reference decoder's
    (stage1_mamba2_config.hpp:211, resolve_secret_key_dist in
    stage1_mamba2_decode_fideslib.cpp:284-291).  security "128-classic": the
    reference's audited classical-128 setting (packed_fideslib.cpp:
    1060-1075, results/b300/2026-09-28/long-accuracy/*/native.json
    security_audit): N=2^17, 65536 slots (batch = ring / 2, as the
    decoder's stage1_mamba2_decode_fideslib.cpp:1005), depth 44, four HYBRID
    digits (45 Q + 12 P primes, QP = 3376 bits against the 3523-bit bound),
    a uniform ternary secret by default, and the audit must pass.  `layers`
    > 0 decodes only the first layers (and the final norm).

    autoregressive: the client-in-loop greedy protocol over the payload's
    autoregressive assets (AutoregressiveAssets; the reference decoder's
    --autoregressive-client-loop): the prompt embeddings, then after each
    evaluation from the last prompt token on the client decrypts, selects
    the greedy token from its logits and encrypts that token's embedding
    next; errors are taken against the assets' polynomial and exact final
    hiddens, and the selected ids against the exporter's greedy ids.

    s2c_first (default): refresh with the SlotToCoeff-first bootstrap (the
    packed executor's --s2c-first circuit; real slots, one EvalMod), about
    40% less bootstrap time than the ordinary order at the same usable
    level interval and precision; False: the ordinary order.  ring_dim
    (not-set only; default 2^16) picks a smaller ring for small payloads."""
    chain, classical, secret_key_dist, slots, extra = _decode_setup(
        payload_dir, security, secret_key_dist, ring_dim, sizes)
    if transient_passes is None:
        transient_passes = default_transient_passes(secret_key_dist, bootstrap_passes)
    n_layers_total = chain.n_layers
    ar = chain.autoregressive if autoregressive else None
    if autoregressive:
        if ar is None:
            raise ValueError("autoregressive client loop requested but the payload has no assets")
        if layers and layers != chain.n_layers:
            raise ValueError("the autoregressive client loop requires the full layer chain")
        if tokens > ar.server_evaluations:
            raise ValueError(f"tokens exceeds the autoregressive server_evaluations "
                             f"({ar.server_evaluations})")
    _truncate(chain, layers)
    n_tok = tokens or (ar.server_evaluations if ar else chain.n_test_tokens)
    if ar is None and n_tok > chain.n_test_tokens:
        raise ValueError("tokens exceeds the payload's n_test_tokens")
    t0 = time.perf_counter()
    cc, keys = _build(slots, seed, secret_key_dist, extra)
    audit = cc.SecurityAudit() if classical else None
    dec = EncryptedMamba2Decoder(cc, keys, chain, bootstrap_passes=bootstrap_passes,
                                 transient_passes=transient_passes, log=log,
                                 s2c_first=s2c_first, level_budget=level_budget)
    setup = time.perf_counter() - t0
    loop = token_loop(dec, chain, n_tok, ar, cc.device.sync, log)
    per_token, errs_poly, errs_exact = loop["seconds"], loop["errors_poly"], loop["errors_exact"]
    selected, client_seconds = loop["selected"], loop["client_seconds"]
    s = dec.ev.stats
    ar_report = {}
    if ar is not None:
        expected = ar.expected_ids[:max(0, n_tok - ar.prompt_tokens + 1)]
        ar_report = {"autoregressive_protocol": "client-in-loop-greedy-v1",
                     "autoregressive_selected_ids": selected,
                     "autoregressive_expected_ids": expected,
                     "autoregressive_tokens_match": selected == expected,
                     "autoregressive_client_seconds": client_seconds}
    return {**ar_report,
        "schema": "fhemamba-m2-decode-result-v1",
        "encrypted": True,
        "layers": chain.n_layers,
        "joint_gate_layers": sum(lay.joint is not None for lay in chain.layers),
        "tokens": n_tok,
        "ring_dimension": cc.GetRingDimension(),
        "slots": slots,
        "security": security,
        "security_audit": audit,
        "s2c_first": s2c_first,
        "secret_key_dist": secret_key_dist,
        "setup_seconds": setup,
        "seconds_per_token": per_token,
        "first_token_seconds": per_token[0],
        "carried_token_seconds": (sum(per_token[1:]) / (n_tok - 1)) if n_tok > 1 else None,
        "max_abs_error_vs_polynomial": max(errs_poly) if errs_poly else None,
        "max_abs_error_vs_exact": max(errs_exact),
        "per_token_errors_vs_polynomial": errs_poly,
        "bootstraps": s["bootstraps"],
        "logical_refreshes": s["logical_refreshes"],
        "bootstrap_seconds": s["bootstrap_seconds"],
        "rotations": s["rotations"],
        "ct_ct_mul": s["ct_ct"],
        "ct_pt_mul": s["ct_pt"],
        "rotation_keys_generated": s["rotation_keys"],
        "keygen_seconds": s["keygen_seconds"],
        "n_layers_total": n_layers_total,
        "per_token_errors_vs_exact": errs_exact,
        "per_token_bootstraps": loop["bootstraps"],
        "token_windows_monotonic_ns": loop["windows_ns"],
        "decrypt_seconds": loop["decrypt_seconds"],
        "token0_samples": loop["token0"],
        "level_budget": list(level_budget),
        "refresh_passes": [dec.critical_passes, dec.transient_passes],
        "multiplicative_depth": len(cc.GetModuli()[0]) - 1,
        "dims": {"d_model": dec.d, "d_inner": dec.di, "num_heads": dec.nh,
                 "head_dim": dec.hd, "state_size": dec.ns, "conv_kernel": dec.kc,
                 "conv_dim": dec.cd, "proj_dim": chain.layers[0].proj_dim,
                 "n_groups": chain.layers[0].n_groups, "state_group_count": dec.groups},
    }


def main(argv=None) -> int:
    import argparse
    import json
    import sys
    ap = argparse.ArgumentParser(description="encrypted Mamba-2 decode of a chain payload")
    ap.add_argument("payload")
    ap.add_argument("result")
    ap.add_argument("--tokens", type=int, default=0)
    ap.add_argument("--bootstrap-passes", type=int, default=2, choices=(1, 2),
                    help="passes of the precision-critical refreshes (carried state, FIFO, "
                         "gated norm input, last residuals, scheduled normalization)")
    ap.add_argument("--transient-passes", type=int, default=None, choices=(1, 2),
                    help="passes of the other refreshes (default: 1 with a sparse-ternary "
                         "secret, else --bootstrap-passes)")
    ap.add_argument("--tolerance", type=float, default=1e-3,
                    help="pass threshold on the error against the polynomial circuit")
    ap.add_argument("--secret-key-dist", default=None, choices=sorted(SECRET_KEY_DISTS),
                    help="default: sparse-ternary, uniform-ternary under 128-classic")
    ap.add_argument("--security", default="not-set", choices=("not-set", "128-classic"))
    ap.add_argument("--layers", type=int, default=0,
                    help="decode only the first LAYERS layers (0: all)")
    ap.add_argument("--autoregressive-client-loop", action="store_true",
                    help="greedy client-in-loop decoding over the payload's assets")
    ap.add_argument("--ordinary-bootstrap", action="store_true",
                    help="refresh with the ordinary bootstrap order instead of SlotToCoeff-first")
    ap.add_argument("--process-role", default="inline",
                    choices=("inline", "client-init", "server-eval", "client-decrypt"),
                    help="process-separated decode through --handoff-dir (fhemamba_amd.handoff)")
    ap.add_argument("--handoff-dir", default="")
    ap.add_argument("--ring-dim", type=int, default=0,
                    help="ring dimension under security not-set (default 65536)")
    args = ap.parse_args(sys.argv[1:] if argv is None else argv)
    if args.process_role != "inline":
        from . import handoff as H
        try:
            if not args.handoff_dir:
                raise ValueError("non-inline process-role requires --handoff-dir")
            if args.autoregressive_client_loop:
                raise ValueError("process-separated autoregressive loop is not implemented")
            if args.process_role == "client-init":
                report = H.client_init(
                    args.payload, args.handoff_dir, tokens=args.tokens,
                    bootstrap_passes=args.bootstrap_passes,
                    transient_passes=args.transient_passes,
                    secret_key_dist=args.secret_key_dist, security=args.security,
                    layers=args.layers, s2c_first=not args.ordinary_bootstrap,
                    ring_dim=args.ring_dim)
            elif args.process_role == "server-eval":
                report = H.server_eval(args.payload, args.handoff_dir, tokens=args.tokens,
                                       layers=args.layers)
            else:
                report = H.client_decrypt(args.payload, args.handoff_dir, tokens=args.tokens,
                                          layers=args.layers, tolerance=args.tolerance)
        except Exception as exc:  # noqa: BLE001 - reported as exit code 2
            print(exc, file=sys.stderr)
            return 2
        with open(args.result, "w") as f:
            json.dump(report, f)
        return 0 if report["passed"] else 1
    try:
        report = run_payload(args.payload, tokens=args.tokens,
                             bootstrap_passes=args.bootstrap_passes,
                             transient_passes=args.transient_passes,
                             secret_key_dist=args.secret_key_dist, security=args.security,
                             layers=args.layers,
                             autoregressive=args.autoregressive_client_loop,
                             s2c_first=not args.ordinary_bootstrap, ring_dim=args.ring_dim)
    except Exception as exc:  # noqa: BLE001 - reported as exit code 2
        print(exc, file=sys.stderr)
        return 2
    err = report["max_abs_error_vs_polynomial"]
    report["passed"] = bool(err is not None and err <= args.tolerance and
                            report.get("autoregressive_tokens_match", True))
    with open(args.result, "w") as f:
        json.dump(report, f)
    return 0 if report["passed"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
