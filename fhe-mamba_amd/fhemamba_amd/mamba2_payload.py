"""Mamba-2 chain payloads: reader, seeded synthetic writer and the plain
references the encrypted decode is checked against.

Format (as native/fideslib_stage0/src/stage1_mamba2_payload.cpp reads it):
  * a chain directory with `chain.json` (format "fhemamba-m2-chain-v1",
    n_layers, n_test_tokens, final_norm_eps, layer_dirs, tensors:
    final_norm_w, chain_input_embeddings, chain_expected_final and
    optionally chain_expected_poly_final) and `<name>.bin` float32-LE
    row-major arrays (:425-470, :128-152);
  * one directory per layer with `meta.json` (format "fhemamba-m1-v1", dims,
    eps {block_norm, gated_norm}, n_test_tokens, polys {conv_silu,
    gate_silu, dt_softplus, decay_exp, rms_invsqrt, gated_rms_invsqrt},
    tensors: in_proj_w, conv_w, conv_b, dt_bias, a_log, d_skip,
    block_norm_w, gated_norm_w, out_proj_w, test_layer_input,
    test_layer_output) and its `.bin` tensors (:233-330).
Polynomial kinds (src/fhemamba/m1_payload.py:379-408 and
src/fhemamba/ops.py:178-459): "cheb" (Chebyshev series on [lo, hi]),
"cheb-squared" (p(x)^2), "cheb-resquared" (p(x / 2^s)^(2^s), optional head
mask), "poly-newton" (y = 0.9 p(v), Newton steps y <- y (1.5 - v y^2 / 2)),
"sq-poly-newton" (y = damping q(v)^2, Newton steps), and the scheduled
normalization recipe "scaled-goldschmidt-invsqrt-v1" for the block, gated
and final norms (chain.json final_norm_poly).  Joint-gate payloads
(layer format "fhemamba-m1-joint-v1", chain format
"fhemamba-m2-chain-joint-v1") carry a "shared-dissipation-factor-v1" gate
that replaces dt_softplus and decay_exp on every head (JointGateSpec).  A
chain.json "autoregressive" block with client_embedding_w (and optionally
client_lm_head_w / _b) holds the client-in-loop greedy assets
(AutoregressiveAssets).

Decode semantics per layer (src/fhemamba/reference.py:182-339, ngroups 1,
no MLP split): hidden -> RMSNorm (rms_invsqrt) -> in_proj -> z | xBC | dt;
causal depthwise conv of xBC over the FIFO of the last conv_kernel - 1
inputs, SiLU (conv_silu); dt = softplus(dt + dt_bias) (dt_softplus),
decay = exp(dt A) (decay_exp), A = -exp(a_log); state update h = decay h +
(dt x) B, readout y = h C + D x; gated = y silu(z) (gate_silu); RMSNorm
with gated_rms_invsqrt and gated_norm_w; out_proj; residual add.  The final
hidden goes through RMSNorm with final_norm_w (the last layer's rms_invsqrt
polynomial).
"""
from __future__ import annotations

import json
import math
import os
from dataclasses import dataclass, field

import numpy as np

SITES = ("conv_silu", "gate_silu", "dt_softplus", "decay_exp", "rms_invsqrt",
         "gated_rms_invsqrt")
LAYER_TENSORS = ("in_proj_w", "conv_w", "conv_b", "dt_bias", "a_log", "d_skip",
                 "block_norm_w", "gated_norm_w", "out_proj_w", "test_layer_input",
                 "test_layer_output")


# ----------------------------------------------------------------- polynomials
@dataclass
class PolySpec:
    kind: str
    coeffs: np.ndarray
    lo: float
    hi: float
    squarings: int = 0
    iterations: int = 0
    damping: float = 1.0
    head_mask: np.ndarray | None = None

    def cheb(self, x):
        t = (2.0 * np.asarray(x, dtype=np.float64) - (self.lo + self.hi)) / (self.hi - self.lo)
        return np.polynomial.chebyshev.chebval(t, self.coeffs)

    def __call__(self, x):
        x = np.asarray(x, dtype=np.float64)
        if self.kind == "cheb":
            return self.cheb(x)
        if self.kind == "cheb-squared":
            y = self.cheb(x)
            return y * y
        if self.kind == "cheb-resquared":
            y = self.cheb(x / 2.0 ** self.squarings)
            for _ in range(self.squarings):
                y = y * y
            return y
        if self.kind in ("poly-newton", "sq-poly-newton"):
            if self.kind == "poly-newton":
                y = 0.9 * self.cheb(x)
            else:
                q = self.cheb(x)
                y = self.damping * q * q
            for _ in range(self.iterations):
                y = y * (1.5 - 0.5 * x * y * y)
            return y
        raise ValueError(f"unsupported polynomial kind: {self.kind}")

    def to_json(self) -> dict:
        d = {"kind": self.kind, "coeffs": [float(c) for c in self.coeffs], "lo": self.lo,
             "hi": self.hi}
        if self.squarings:
            d["squarings"] = self.squarings
        if self.iterations:
            d["iterations"] = self.iterations
        if self.kind in ("poly-newton", "sq-poly-newton"):
            d["damping"] = self.damping
        if self.head_mask is not None:
            d["head_mask"] = [float(v) for v in self.head_mask]
        return d

    @classmethod
    def from_json(cls, d: dict) -> "PolySpec":
        kind = d["kind"]
        if kind not in ("cheb", "cheb-squared", "cheb-resquared", "poly-newton",
                        "sq-poly-newton"):
            raise ValueError(f"unsupported polynomial kind: {kind}")
        mask = d.get("head_mask")
        return cls(kind, np.asarray(d["coeffs"], dtype=np.float64), float(d["lo"]),
                   float(d["hi"]), int(d.get("squarings", 0)), int(d.get("iterations", 0)),
                   float(d.get("damping", 1.0)),
                   None if mask is None else np.asarray(mask, dtype=np.float64))


@dataclass
class ScheduledInvSqrtSpec:
    """Scheduled normalization ("scaled-goldschmidt-invsqrt-v1"): a public
    schedule of Goldschmidt stages and one final recomputed Newton step,
    the recipe the reference exports (src/fhemamba/normalization.py:40-91,
    read by native/fideslib_stage0/src/stage1_mamba2_payload.cpp:437-441):
      u = v seed^2, y = seed;
      per stage (a, b): f = a - b u, y <- y f, u <- u f^2 (not after the
      last stage);
      y <- y (1.5 - 0.5 v y^2).
    Evaluated in float64, as the recipe's oracle workspace."""
    lo: float
    hi: float
    seed: float
    coefficients: tuple
    tolerance: float
    kind: str = "scaled-goldschmidt-invsqrt-v1"

    def __call__(self, v):
        v = np.asarray(v, dtype=np.float64)
        u = v * self.seed * self.seed
        y = self.seed
        n = len(self.coefficients)
        for i, (a, b) in enumerate(self.coefficients):
            f = a - b * u
            y = y * f
            if i + 1 < n:
                u = u * (f * f)
        return y * (1.5 - 0.5 * (v * (y * y)))

    def to_json(self) -> dict:
        return {"kind": self.kind, "lo": self.lo, "hi": self.hi, "seed": self.seed,
                "coefficients": [list(p) for p in self.coefficients],
                "tolerance": self.tolerance, "final_recomputed_newton": True,
                "oracle_workspace_dtype": "float64"}

    @classmethod
    def from_json(cls, d: dict) -> "ScheduledInvSqrtSpec":
        """The reference's recipe check (normalization.py:142-155, :55-63)."""
        if (d.get("kind") != "scaled-goldschmidt-invsqrt-v1"
                or d.get("final_recomputed_newton") is not True
                or d.get("oracle_workspace_dtype") != "float64"):
            raise ValueError("unsupported inverse-square-root recipe")
        coeffs = tuple((float(a), float(b)) for a, b in d["coefficients"])
        lo, hi, seed, tol = (float(d[k]) for k in ("lo", "hi", "seed", "tolerance"))
        vals = [lo, hi, seed, tol] + [x for pr in coeffs for x in pr]
        if not all(math.isfinite(x) for x in vals) or not 0 < lo < hi or not seed > 0 \
                or not 0 < tol < 1 or not coeffs:
            raise ValueError("invalid inverse-square-root schedule")
        return cls(lo, hi, seed, coeffs, tol)


@dataclass
class JointGateSpec:
    """Joint selective gate ("shared-dissipation-factor-v1"): per head h a
    public domain [lo_h, hi_h] and two Chebyshev series p_h, q_h whose
    coefficient matrices are stored degree-major, head-minor.  For
    z = dt + dt_bias,
      t = (2 z - (lo + hi)) / (hi - lo),  p = sum_i p[i, h] T_i(t),
      q likewise,  write = p^2 q^2,  decay = 1 - p^2;
    write takes the place of dt in the state update (h = decay h +
    (write x) B).  Semantics of src/fhemamba/selective_gates.py:113-135 and
    ops.py:553-571; payload checks of
    native/fideslib_stage0/include/stage1_joint_gates.hpp:51-66 and
    src/stage1_mamba2_payload.cpp:208-230.  Evaluated in float64."""
    lo: np.ndarray
    hi: np.ndarray
    p: np.ndarray            # [degree_p + 1][heads]
    q: np.ndarray            # [degree_q + 1][heads]
    rates: np.ndarray
    kind: str = "shared-dissipation-factor-v1"

    @property
    def heads(self) -> int:
        return len(self.lo)

    @property
    def degree(self) -> int:
        """The larger of the two series' degrees (the shared basis size)."""
        return max(len(self.p), len(self.q)) - 1

    def roots(self, z):
        """(p, q) for z of shape [..., heads]."""
        z = np.asarray(z, dtype=np.float64)
        t = (2.0 * z - (self.lo + self.hi)) / (self.hi - self.lo)
        cv = np.polynomial.chebyshev.chebval
        p = np.stack([cv(t[..., h], self.p[:, h]) for h in range(self.heads)], axis=-1)
        q = np.stack([cv(t[..., h], self.q[:, h]) for h in range(self.heads)], axis=-1)
        return p, q

    def __call__(self, z):
        """(write, decay) for z = dt + dt_bias."""
        p, q = self.roots(z)
        d = p * p
        return d * (q * q), 1.0 - d

    def bounds(self) -> tuple:
        """Certified maxima of |write| and |decay| for z inside every head's
        domain (|T_i| <= 1 on [-1, 1])."""
        pm = np.abs(self.p).sum(axis=0)
        qm = np.abs(self.q).sum(axis=0)
        return float(np.max(pm * pm * qm * qm)), float(max(1.0, np.max(pm * pm - 1.0)))

    def to_json(self) -> dict:
        return {"kind": self.kind, "lo": list(self.lo), "hi": list(self.hi),
                "p": list(self.p.reshape(-1)), "q": list(self.q.reshape(-1)),
                "rates": list(self.rates), "coefficient_layout": "degree-major-head-minor",
                "all_heads_retained": True}

    @classmethod
    def from_json(cls, d: dict, heads: int) -> "JointGateSpec":
        if d.get("kind") != "shared-dissipation-factor-v1" or \
                d.get("coefficient_layout") != "degree-major-head-minor":
            raise ValueError("unsupported joint gate recipe")
        arrays = {}
        for name in ("lo", "hi", "p", "q", "rates"):
            v = d.get(name)
            if not isinstance(v, list) or not v or \
                    not all(isinstance(x, (int, float)) and not isinstance(x, bool) for x in v):
                raise ValueError("invalid joint gate numeric array")
            arrays[name] = np.asarray(v, dtype=np.float64)
            if not np.all(np.isfinite(arrays[name])):
                raise ValueError("joint gate contains non-finite values")
        lo, hi, rates = arrays["lo"], arrays["hi"], arrays["rates"]
        if heads < 1 or len(lo) != heads or len(hi) != heads or len(rates) != heads:
            raise ValueError("joint gate requires one domain/rate per head")
        if np.any(lo >= hi) or np.any(rates <= 0):
            raise ValueError("invalid joint gate domain/rate")
        mats = []
        for name in ("p", "q"):
            c = arrays[name]
            if len(c) % heads or len(c) // heads > 4097:
                raise ValueError("invalid joint gate coefficient matrix shape")
            mats.append(c.reshape(-1, heads))
        return cls(lo, hi, mats[0], mats[1], rates)


def read_poly(d: dict):
    """A site's polynomial spec: a Chebyshev-based PolySpec or a scheduled
    inverse square root."""
    if d.get("kind") == "scaled-goldschmidt-invsqrt-v1":
        return ScheduledInvSqrtSpec.from_json(d)
    return PolySpec.from_json(d)


def fit_chebyshev(fn, lo: float, hi: float, degree: int) -> np.ndarray:
    """Least-squares Chebyshev fit of fn on [lo, hi] at Chebyshev points."""
    if not hi > lo:
        raise ValueError(f"invalid fit interval [{lo}, {hi}]")
    m = max(4 * (degree + 1), 256)
    t = np.cos(np.pi * (np.arange(m) + 0.5) / m)
    x = 0.5 * (t + 1.0) * (hi - lo) + lo
    return np.polynomial.chebyshev.chebfit(t, fn(x), degree)


def silu(x):
    return x / (1.0 + np.exp(-x))


def softplus(x):
    return np.logaddexp(0.0, x)


# ----------------------------------------------------------------- payload
@dataclass
class LayerPayload:
    d_model: int
    d_inner: int
    num_heads: int
    head_dim: int
    state_size: int
    n_groups: int
    conv_kernel: int
    conv_dim: int
    eps_block: float
    eps_gated: float
    n_test_tokens: int
    polys: dict
    tensors: dict
    bounds: dict = field(default_factory=dict)   # calibration |value| maxima by checkpoint
    joint: JointGateSpec | None = None           # joint gate (replaces dt_softplus, decay_exp)

    @property
    def proj_dim(self) -> int:
        return 2 * self.d_inner + 2 * self.n_groups * self.state_size + self.num_heads

    def t(self, name):
        return self.tensors[name]


@dataclass
class ChainPayload:
    n_layers: int
    n_test_tokens: int
    final_norm_eps: float
    final_norm_w: np.ndarray
    input_embeddings: np.ndarray
    expected_final: np.ndarray
    expected_poly_final: np.ndarray | None
    layers: list = field(default_factory=list)
    # dedicated final-norm inverse square root (scheduled payloads); None:
    # the last layer's rms_invsqrt (m1_payload.py:421-426)
    final_norm_poly: object = None

    # client-in-loop greedy assets (chain.json "autoregressive"); None: none
    autoregressive: "AutoregressiveAssets | None" = None

    def final_invsqrt(self):
        return self.final_norm_poly or self.layers[-1].polys["rms_invsqrt"]


@dataclass
class AutoregressiveAssets:
    """Client-in-loop greedy decoding ("client-in-loop-greedy-v1"): the
    server evaluates prompt_tokens + generate_tokens - 1 embeddings; after
    each evaluation from the last prompt token on, the client decrypts the
    final normed hidden, takes logits = lm_head_w hidden (+ lm_head_b; the
    embedding table when the two are tied), selects the first maximal logit
    and sends that token's embedding next (src/fhemamba/m1_payload.py:
    519-618 writes the assets, native/fideslib_stage0/src/
    stage1_mamba2_payload.cpp:476-528 reads them and
    stage1_mamba2_decode_fideslib.cpp:4549-4611 runs the client step)."""
    prompt_tokens: int
    generate_tokens: int
    server_evaluations: int
    prompt_ids: list
    expected_ids: list               # poly_generated_ids: the pass criterion
    embedding_w: np.ndarray          # [vocab][d_model]
    lm_head_w: np.ndarray | None     # None: tied to embedding_w
    lm_head_b: np.ndarray | None
    embeddings: np.ndarray           # [server_evaluations][d_model]
    expected_poly_final: np.ndarray
    expected_exact_final: np.ndarray

    @property
    def vocab(self) -> int:
        return self.embedding_w.shape[0]

    def select(self, hidden) -> int:
        """The client's greedy choice for a decrypted final hidden."""
        w = self.embedding_w if self.lm_head_w is None else self.lm_head_w
        with np.errstate(invalid="ignore", over="ignore"):
            logits = w @ np.asarray(hidden, dtype=np.float64)
            if self.lm_head_b is not None:
                logits = logits + self.lm_head_b
        if not np.all(np.isfinite(logits)):
            raise ValueError("non-finite autoregressive client logit")
        return int(np.argmax(logits))

    def input_for(self, step: int, selected: list) -> np.ndarray:
        """The embedding evaluated at `step`: the prompt's, then the client's
        previous choice."""
        if step < self.prompt_tokens:
            return self.embeddings[step]
        if len(selected) != step - self.prompt_tokens + 1:
            raise ValueError("missing client-selected autoregressive embedding")
        return self.embedding_w[selected[-1]]


def _read_bin(path: str, shape) -> np.ndarray:
    count = int(np.prod(shape)) if len(shape) else 1
    size = os.path.getsize(path)
    if size != 4 * count:
        raise ValueError(f"tensor size mismatch for {os.path.basename(path)}: expected "
                         f"{4 * count} bytes, found {size}")
    return np.fromfile(path, dtype="<f4").astype(np.float64).reshape(shape)


def read_layer_payload(directory: str) -> LayerPayload:
    with open(os.path.join(directory, "meta.json")) as f:
        meta = json.load(f)
    fmt = meta.get("format")
    joint = fmt == "fhemamba-m1-joint-v1"
    if fmt != "fhemamba-m1-v1" and not joint:
        raise ValueError("unexpected payload format (want fhemamba-m1-v1)")
    if not joint and "joint_gates" in meta:
        raise ValueError("joint gate payload requires the versioned joint format")
    d, eps = meta["dims"], meta["eps"]
    polys = {}
    for name in SITES:
        spec = meta["polys"][name]
        if spec.get("kind") == "scaled-goldschmidt-invsqrt-v1" and \
                name not in ("rms_invsqrt", "gated_rms_invsqrt"):
            raise ValueError(f"a scheduled inverse square root cannot serve {name}")
        polys[name] = read_poly(spec)
    tensors = {name: _read_bin(os.path.join(directory, name + ".bin"), meta["tensors"][name])
               for name in LAYER_TENSORS}
    layer = LayerPayload(int(d["d_model"]), int(d["d_inner"]), int(d["num_heads"]),
                         int(d["head_dim"]), int(d["state_size"]), int(d["n_groups"]),
                         int(d["conv_kernel"]), int(d["conv_dim"]), float(eps["block_norm"]),
                         float(eps["gated_norm"]), int(meta["n_test_tokens"]), polys, tensors)
    carried = meta.get("carried_bounds") or {}
    # maxima measured on the evaluation prompt itself are not trusted
    # (stage1_mamba2_payload.cpp:253-260)
    if carried.get("source") == "calibration_text":
        layer.bounds = {k: float(v) for k, v in carried.get("checkpoint_abs_max", {}).items()}
    if layer.n_groups != 1:
        raise ValueError("the decoder supports one B/C group")
    if layer.conv_dim != layer.d_inner + 2 * layer.state_size:
        raise ValueError("conv_dim must be d_inner + 2 * state_size")
    mask = getattr(polys["decay_exp"], "head_mask", None)
    if mask is not None and (len(mask) != layer.num_heads or
                             not np.all((mask == 0) | (mask == 1))):
        raise ValueError("decay_exp head_mask must hold one 0/1 value per head")
    if joint:
        layer.joint = JointGateSpec.from_json(meta.get("joint_gates") or {}, layer.num_heads)
        if mask is not None and np.any(mask != 1):
            raise ValueError("joint gates retain all heads")
        # the gate's rates are the layer's -A (ops.py:557-560)
        if not np.allclose(np.exp(layer.t("a_log")), layer.joint.rates, rtol=2e-7, atol=0):
            raise ValueError("joint gate rates differ from the layer's A")
    if layer.t("in_proj_w").shape != (layer.proj_dim, layer.d_model):
        raise ValueError("in_proj_w shape does not match the dims")
    return layer


def read_chain_payload(directory: str) -> ChainPayload:
    with open(os.path.join(directory, "chain.json")) as f:
        meta = json.load(f)
    if meta.get("format") not in ("fhemamba-m2-chain-v1", "fhemamba-m2-chain-joint-v1"):
        raise ValueError("unexpected chain payload format (want fhemamba-m2-chain-v1)")
    n_layers = int(meta["n_layers"])
    dirs = meta["layer_dirs"]
    if n_layers <= 0 or len(dirs) != n_layers:
        raise ValueError("chain.json layer_dirs does not match n_layers")
    tens = meta["tensors"]

    def rb(name):
        return _read_bin(os.path.join(directory, name + ".bin"), tens[name])

    chain = ChainPayload(n_layers, int(meta["n_test_tokens"]), float(meta["final_norm_eps"]),
                         rb("final_norm_w"), rb("chain_input_embeddings"),
                         rb("chain_expected_final"),
                         rb("chain_expected_poly_final") if "chain_expected_poly_final" in tens
                         else None)
    chain.layers = [read_layer_payload(os.path.join(directory, d)) for d in dirs]
    if meta.get("final_norm_poly") is not None:
        chain.final_norm_poly = read_poly(meta["final_norm_poly"])
    if isinstance(meta.get("autoregressive"), dict):
        chain.autoregressive = _read_autoregressive(meta["autoregressive"], tens, rb,
                                                    chain.layers[0].d_model)
    first = chain.layers[0]
    for i, lay in enumerate(chain.layers):
        if (lay.d_model, lay.d_inner, lay.num_heads, lay.head_dim, lay.state_size,
                lay.conv_kernel) != (first.d_model, first.d_inner, first.num_heads,
                                     first.head_dim, first.state_size, first.conv_kernel):
            raise ValueError(f"chain layer payload dims mismatch at index {i}")
    return chain


def _read_autoregressive(ar: dict, tens: dict, rb, d_model: int) -> AutoregressiveAssets:
    """Checks of stage1_mamba2_payload.cpp:476-528 and
    stage1_mamba2_decode_fideslib.cpp:791-876."""
    if ar.get("protocol") != "client-in-loop-greedy-v1":
        raise ValueError("unsupported autoregressive payload protocol")
    pt, gt, ev = (int(ar[k]) for k in ("prompt_tokens", "generate_tokens",
                                        "server_evaluations"))
    if pt < 1 or gt < 1 or ev != pt + gt - 1:
        raise ValueError("invalid autoregressive evaluation count")
    ids = [int(v) for v in ar.get("poly_generated_ids", [])]
    emb = rb("client_embedding_w")
    if emb.ndim != 2 or emb.shape[1] != d_model:
        raise ValueError("client_embedding_w must be rank 2 with d_model columns")
    vocab = emb.shape[0]
    head = rb("client_lm_head_w") if "client_lm_head_w" in tens else None
    bias = rb("client_lm_head_b") if "client_lm_head_b" in tens else None
    assets = AutoregressiveAssets(
        pt, gt, ev, [int(v) for v in ar.get("prompt_ids", [])], ids, emb, head, bias,
        rb("autoregressive_poly_embeddings"), rb("autoregressive_poly_expected_final"),
        rb("autoregressive_exact_expected_final"))
    if len(ids) != gt or any(not 0 <= i < vocab for i in ids) or \
            (head is not None and head.shape != (vocab, d_model)) or \
            (bias is not None and bias.shape != (vocab,)) or \
            any(a.shape != (ev, d_model) for a in (assets.embeddings,
                                                   assets.expected_poly_final,
                                                   assets.expected_exact_final)):
        raise ValueError("autoregressive tensor shape mismatch")
    return assets


# ----------------------------------------------------------------- plain decode
@dataclass
class LayerState:
    ssm: np.ndarray          # [heads][head_dim][state]
    fifo: list               # last conv_kernel - 1 xBC vectors, oldest first


def zero_state(lay: LayerPayload) -> LayerState:
    return LayerState(np.zeros((lay.num_heads, lay.head_dim, lay.state_size)),
                      [np.zeros(lay.conv_dim) for _ in range(lay.conv_kernel - 1)])


def rms_inv(v, poly: PolySpec | None):
    return 1.0 / np.sqrt(v) if poly is None else poly(v)


def layer_step(lay: LayerPayload, hidden: np.ndarray, state: LayerState, polynomial: bool):
    """One token through one layer: (new hidden, new state).  polynomial=True
    evaluates every nonlinearity with the payload's polynomials (the circuit
    the encrypted decode runs), False with the exact functions."""
    P = lay.polys if polynomial else {}
    di, ns, nh, hd = lay.d_inner, lay.state_size, lay.num_heads, lay.head_dim
    v = np.mean(hidden ** 2) + lay.eps_block
    normed = hidden * rms_inv(v, P.get("rms_invsqrt")) * lay.t("block_norm_w")
    proj = lay.t("in_proj_w") @ normed
    z, xbc, dt_raw = proj[:di], proj[di:di + lay.conv_dim], proj[di + lay.conv_dim:]
    window = state.fifo + [xbc]                             # oldest first, current last
    conv = sum(lay.t("conv_w")[:, k] * window[k] for k in range(lay.conv_kernel)) + \
        lay.t("conv_b")
    act = P["conv_silu"](conv) if polynomial else silu(conv)
    x, B, C = act[:di], act[di:di + ns], act[di + ns:]
    t = dt_raw + lay.t("dt_bias")
    A = -np.exp(lay.t("a_log"))
    if polynomial and lay.joint is not None:
        dt, decay = lay.joint(t)
    elif polynomial:
        dt = P["dt_softplus"](t)
        decay = P["decay_exp"](dt * A)
        mask = P["decay_exp"].head_mask
        if mask is not None:
            decay = decay * mask
    else:
        dt = softplus(t)
        decay = np.exp(dt * A)
    xh = x.reshape(nh, hd)
    h = decay[:, None, None] * state.ssm + (dt[:, None] * xh)[:, :, None] * B[None, None, :]
    y = np.einsum("hpn,n->hp", h, C) + lay.t("d_skip")[:, None] * xh
    g = P["gate_silu"](z) if polynomial else silu(z)
    gated = y.reshape(-1) * g
    v2 = np.mean(gated ** 2) + lay.eps_gated
    yn = gated * rms_inv(v2, P.get("gated_rms_invsqrt")) * lay.t("gated_norm_w")
    out = hidden + lay.t("out_proj_w") @ yn
    return out, LayerState(h, window[1:])


def final_norm(chain: ChainPayload, hidden: np.ndarray, polynomial: bool):
    v = np.mean(hidden ** 2) + chain.final_norm_eps
    poly = chain.final_invsqrt() if polynomial else None
    return hidden * rms_inv(v, poly) * chain.final_norm_w


def autoregressive_decode(chain: ChainPayload, polynomial: bool, evaluations: int = 0):
    """The client-in-loop greedy protocol on the plain decode: (final
    hiddens [evaluations][d_model], selected ids)."""
    ar = chain.autoregressive
    if ar is None:
        raise ValueError("the payload has no autoregressive assets")
    n = evaluations or ar.server_evaluations
    if not 1 <= n <= ar.server_evaluations:
        raise ValueError("evaluations exceed the payload's server_evaluations")
    states = [zero_state(lay) for lay in chain.layers]
    finals, selected = [], []
    for step in range(n):
        h = ar.input_for(step, selected)
        for i, lay in enumerate(chain.layers):
            h, states[i] = layer_step(lay, h, states[i], polynomial)
        finals.append(final_norm(chain, h, polynomial))
        if step >= ar.prompt_tokens - 1:
            selected.append(ar.select(finals[-1]))
    return np.array(finals), selected


def decode_tokens(chain: ChainPayload, embeddings: np.ndarray, polynomial: bool,
                  states=None):
    """Decode each embedding in turn from `states` (zero by default);
    returns (final normed hidden per token [tokens][d_model], states)."""
    states = states or [zero_state(lay) for lay in chain.layers]
    outs = []
    for e in np.asarray(embeddings):
        h = e
        for i, lay in enumerate(chain.layers):
            h, states[i] = layer_step(lay, h, states[i], polynomial)
        outs.append(final_norm(chain, h, polynomial))
    return np.array(outs), states


# ----------------------------------------------------------------- synthetic
MAMBA2_130M = dict(d_model=768, d_inner=1536, num_heads=24, head_dim=64, state_size=128,
                   conv_kernel=4, n_layers=24)
DEGREES = {"conv_silu": 96, "gate_silu": 64, "dt_softplus": 64, "decay_exp": 24,
           "rms_invsqrt": 47, "gated_rms_invsqrt": 31}


def _write_bin(directory, name, arr, manifest):
    arr = np.asarray(arr, dtype="<f4")
    arr.tofile(os.path.join(directory, name + ".bin"))
    manifest[name] = list(arr.shape)


def synthetic_chain(directory: str, *, seed: int = 0, n_layers: int = 24, n_test_tokens: int = 2,
                    d_model: int = 768, d_inner: int = 1536, num_heads: int = 24,
                    head_dim: int = 64, state_size: int = 128, conv_kernel: int = 4,
                    degrees=None, calibration_tokens: int = 8,
                    joint_degrees: tuple | None = None) -> ChainPayload:
    """Write a chain payload for a random-init Mamba-2 model of the given
    shape (weights N(0, 0.02), A = -exp(U[0, ln 16]), dt_bias so that dt
    starts in [0.001, 0.1], D = 1, norm weights 1): polynomial intervals come
    from an exact plain decode of `calibration_tokens` random embeddings,
    widened by 30%, and the test vectors from a separate draw.

    joint_degrees = (degree_p, degree_q) writes joint-gate payloads instead
    (_fit_joint_gate): per head, on that head's widened range of
    dt + dt_bias, p fits sqrt(1 - exp(dt A)) and q fits
    sqrt(dt / (1 - exp(dt A))), so that write = p^2 q^2 ~ dt and
    decay = 1 - p^2 ~ exp(dt A)."""
    degrees = dict(DEGREES, **(degrees or {}))
    rng = np.random.default_rng(seed)
    os.makedirs(directory, exist_ok=True)
    conv_dim = d_inner + 2 * state_size
    proj_dim = 2 * d_inner + 2 * state_size + num_heads
    layers = []
    for _ in range(n_layers):
        dt0 = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), num_heads))
        tensors = {
            "in_proj_w": rng.normal(0, 0.02, (proj_dim, d_model)),
            "conv_w": rng.normal(0, 0.2, (conv_dim, conv_kernel)),
            "conv_b": rng.normal(0, 0.02, conv_dim),
            "dt_bias": dt0 + np.log(-np.expm1(-dt0)),
            "a_log": np.log(rng.uniform(1, 16, num_heads)),
            "d_skip": np.ones(num_heads),
            "block_norm_w": np.ones(d_model),
            "gated_norm_w": np.ones(d_inner),
            "out_proj_w": rng.normal(0, 0.02, (d_model, d_inner)),
        }
        # the payload stores float32: calibrate and reference on those values
        tensors = {k: v.astype(np.float32).astype(np.float64) for k, v in tensors.items()}
        layers.append(LayerPayload(d_model, d_inner, num_heads, head_dim, state_size, 1,
                                   conv_kernel, conv_dim, 1e-5, 1e-5, n_test_tokens, {},
                                   tensors))
    # calibration: record each site's input range on an exact decode
    ranges = [{s: [np.inf, -np.inf] for s in SITES} for _ in layers]
    peaks: list = [{} for _ in layers]
    states = [zero_state(lay) for lay in layers]
    for e in rng.normal(0, 1, (calibration_tokens, d_model)):
        h = e
        for i, lay in enumerate(layers):
            h, states[i] = _calibrated_step(lay, h, states[i], ranges[i], peaks[i])
    for i, lay in enumerate(layers):
        lay.polys = _fit_layer_polys(ranges[i], lay, degrees)
        lay.bounds = peaks[i]
        if joint_degrees is not None:
            lay.joint = _fit_joint_gate(lay, ranges[i]["t_heads"], *joint_degrees)
    chain = ChainPayload(n_layers, n_test_tokens, 1e-5, np.ones(d_model),
                         rng.normal(0, 1, (n_test_tokens, d_model)).astype(np.float32)
                         .astype(np.float64), None, None, layers)
    # per-layer test vectors and the chain's references (zero initial state)
    states = [zero_state(lay) for lay in layers]
    ins = [[] for _ in layers]
    outs = [[] for _ in layers]
    for e in chain.input_embeddings:
        h = e
        for i, lay in enumerate(layers):
            ins[i].append(h)
            h, states[i] = layer_step(lay, h, states[i], False)
            outs[i].append(h)
    for i, lay in enumerate(layers):
        lay.tensors["test_layer_input"] = np.array(ins[i])
        lay.tensors["test_layer_output"] = np.array(outs[i])
    chain.expected_final, _ = decode_tokens(chain, chain.input_embeddings, False)
    chain.expected_poly_final, _ = decode_tokens(chain, chain.input_embeddings, True)
    write_chain_payload(directory, chain)
    return read_chain_payload(directory)


def _calibrated_step(lay, hidden, state, rng_, peak):
    """Exact step recording each polynomial site's input range and the
    magnitude of every value the encrypted decoder refreshes."""
    def rec(site, v):
        r = rng_[site]
        r[0], r[1] = min(r[0], float(np.min(v))), max(r[1], float(np.max(v)))

    def top(name, v):
        peak[name] = max(peak.get(name, 0.0), float(np.max(np.abs(v))))

    di, ns = lay.d_inner, lay.state_size
    top("residual", hidden)
    v = np.mean(hidden ** 2) + lay.eps_block
    rec("rms_invsqrt", v)
    top("variance", v)
    top("inv", 1.0 / np.sqrt(v))
    raw = lay.t("in_proj_w") @ (hidden * lay.t("block_norm_w"))
    top("proj_raw", raw)
    proj = raw / np.sqrt(v)
    top("proj", proj)
    z, xbc, dt_raw = proj[:di], proj[di:di + lay.conv_dim], proj[di + lay.conv_dim:]
    window = state.fifo + [xbc]
    conv = sum(lay.t("conv_w")[:, k] * window[k] for k in range(lay.conv_kernel)) + \
        lay.t("conv_b")
    rec("conv_silu", conv)
    top("conv", conv)
    act = silu(conv)
    top("act", act)
    x, B, C = act[:di], act[di:di + ns], act[di + ns:]
    t = dt_raw + lay.t("dt_bias")
    rec("dt_softplus", t)
    th = rng_.setdefault("t_heads", [np.full(len(t), np.inf), np.full(len(t), -np.inf)])
    th[0], th[1] = np.minimum(th[0], t), np.maximum(th[1], t)
    dt = softplus(t)
    top("dt", dt)
    A = -np.exp(lay.t("a_log"))
    rec("decay_exp", dt * A)
    nh, hd = lay.num_heads, lay.head_dim
    xh = x.reshape(nh, hd)
    h = np.exp(dt * A)[:, None, None] * state.ssm + (dt[:, None] * xh)[:, :, None] * B
    top("state", h)
    y = np.einsum("hpn,n->hp", h, C) + lay.t("d_skip")[:, None] * xh
    top("y", y)
    rec("gate_silu", z)
    top("gate", silu(z))
    gated = y.reshape(-1) * silu(z)
    top("gated", gated)
    v2 = np.mean(gated ** 2) + lay.eps_gated
    rec("gated_rms_invsqrt", v2)
    top("gated_variance", v2)
    top("gated_inv", 1.0 / np.sqrt(v2))
    oraw = lay.t("out_proj_w") @ (gated * lay.t("gated_norm_w"))
    top("out_raw", oraw)
    out = hidden + oraw / np.sqrt(v2)
    top("output", oraw / np.sqrt(v2))
    vo = np.mean(out ** 2)
    top("out_residual", out)
    top("out_variance", vo)
    top("out_inv", 1.0 / np.sqrt(vo))
    return out, LayerState(h, window[1:])


def _fit_layer_polys(r, lay, degrees) -> dict:
    def widen(site, margin=0.3):
        lo, hi = r[site]
        pad = margin * max(hi - lo, 1e-3)
        return lo - pad, hi + pad

    polys = {}
    for site in ("conv_silu", "gate_silu"):
        lo, hi = widen(site)
        polys[site] = PolySpec("cheb", fit_chebyshev(silu, lo, hi, degrees[site]), lo, hi)
    lo, hi = widen("dt_softplus")
    polys["dt_softplus"] = PolySpec("cheb-squared", fit_chebyshev(
        lambda t: np.sqrt(softplus(t)), lo, hi, degrees["dt_softplus"]), lo, hi)
    lo = min(r["decay_exp"][0] * 1.3, -1e-6)
    s = max(0, math.ceil(math.log2(max(-lo, 1e-9) / 8.0)))
    base_lo = lo / 2 ** s
    polys["decay_exp"] = PolySpec("cheb-resquared", fit_chebyshev(
        np.exp, base_lo, 0.0, degrees["decay_exp"]), base_lo, 0.0, squarings=s,
        head_mask=np.ones(lay.num_heads))
    lo, hi = r["rms_invsqrt"]
    polys["rms_invsqrt"] = PolySpec("poly-newton", fit_chebyshev(
        lambda v: 1.0 / np.sqrt(v), 0.1 * lo, 2.0 * hi, degrees["rms_invsqrt"]),
        0.1 * lo, 2.0 * hi, iterations=4, damping=0.9)
    lo, hi = r["gated_rms_invsqrt"]
    polys["gated_rms_invsqrt"] = PolySpec("sq-poly-newton", fit_chebyshev(
        lambda v: np.abs(v) ** -0.25, 0.02 * lo, 2.0 * hi, degrees["gated_rms_invsqrt"]),
        0.02 * lo, 2.0 * hi, iterations=4, damping=0.85)
    return polys


def _fit_joint_gate(lay, t_range, degree_p: int, degree_q: int) -> JointGateSpec:
    lo_t, hi_t = t_range
    pad = 0.3 * np.maximum(hi_t - lo_t, 1e-3)
    lo, hi = lo_t - pad, hi_t + pad
    rates = np.exp(lay.t("a_log"))
    p = np.zeros((degree_p + 1, lay.num_heads))
    q = np.zeros((degree_q + 1, lay.num_heads))
    for h in range(lay.num_heads):
        def keep(z, h=h):
            return -np.expm1(-softplus(z) * rates[h])      # 1 - exp(dt A) > 0
        p[:, h] = fit_chebyshev(lambda z: np.sqrt(keep(z)), lo[h], hi[h], degree_p)
        q[:, h] = fit_chebyshev(lambda z: np.sqrt(softplus(z) / keep(z)), lo[h], hi[h],
                                degree_q)
    return JointGateSpec(lo, hi, p, q, rates)


def write_chain_payload(directory: str, chain: ChainPayload) -> None:
    os.makedirs(directory, exist_ok=True)
    dirs = []
    for i, lay in enumerate(chain.layers):
        name = f"layer_{i:02d}"
        ld = os.path.join(directory, name)
        os.makedirs(ld, exist_ok=True)
        manifest: dict = {}
        for t in LAYER_TENSORS:
            _write_bin(ld, t, lay.tensors[t], manifest)
        meta = {"format": "fhemamba-m1-v1" if lay.joint is None else "fhemamba-m1-joint-v1",
                "layer_index": i,
                "dims": {"d_model": lay.d_model, "d_inner": lay.d_inner,
                         "num_heads": lay.num_heads, "head_dim": lay.head_dim,
                         "state_size": lay.state_size, "n_groups": lay.n_groups,
                         "conv_kernel": lay.conv_kernel, "conv_dim": lay.conv_dim},
                "eps": {"block_norm": lay.eps_block, "gated_norm": lay.eps_gated},
                "n_test_tokens": lay.n_test_tokens,
                "polys": {k: v.to_json() for k, v in lay.polys.items()},
                "carried_bounds": {"source": "calibration_text",
                                   "checkpoint_abs_max": lay.bounds},
                "tensors": manifest}
        if lay.joint is not None:
            meta["joint_gates"] = lay.joint.to_json()
        with open(os.path.join(ld, "meta.json"), "w") as f:
            json.dump(meta, f)
        dirs.append(name)
    manifest = {}
    _write_bin(directory, "final_norm_w", chain.final_norm_w, manifest)
    _write_bin(directory, "chain_input_embeddings", chain.input_embeddings, manifest)
    _write_bin(directory, "chain_expected_final", chain.expected_final, manifest)
    if chain.expected_poly_final is not None:
        _write_bin(directory, "chain_expected_poly_final", chain.expected_poly_final, manifest)
    with open(os.path.join(directory, "chain.json"), "w") as f:
        joint = any(lay.joint is not None for lay in chain.layers)
        json.dump({"format": "fhemamba-m2-chain-joint-v1" if joint else "fhemamba-m2-chain-v1",
                   "n_layers": chain.n_layers,
                   "n_test_tokens": chain.n_test_tokens,
                   "final_norm_eps": chain.final_norm_eps, "layer_dirs": dirs,
                   "tensors": manifest}, f)
