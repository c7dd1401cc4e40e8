"""CPU oracle: numpy restatement of the reference's decode-step token selection.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg import this module, and only as the checker.

Functions and the reference lines they restate:

* ``rms_norm``            -- nanovllm_jax/layers.py:11-29 (fp32, ``x*rsqrt(mean(x^2)+eps)*(1+w)``).
* ``lm_head_logits``      -- nanovllm_jax/model.py:765-780, 87-102, 400-416
  (``jnp.dot(hidden_norm, W)``: fp32 accumulate; bf16 x bf16 rounds the
  logits to bf16, model.py:806-819 and the Triton ``REDUCE_CAST`` at
  nanovllm_jax/kernels/lm_head_triton.py:58-63, 146-150).
* ``greedy_top1``         -- model.py:819, 894 and lm_head_triton.py:66-75, 99-102
  (maximum value, lowest index among ties; ``jnp.argmax`` lets the first NaN win).
* ``sample_row``          -- model.py:929-938 for the temperature route
  (``T <= 0`` -> argmax, else ``categorical(key, l / max(T, 1e-6))``), extended
  with the top-k / top-p filter that the reference only specifies on paper
  (docs/kernel_roadmap.md:436-446) and in its legacy draft sampler
  (nanovllm_jax/spec_decode.py:69-83): T-scale, keep ``x >= kth_largest(x)``,
  then over the survivors keep ``p >= sorted_p[cutoff]`` with
  ``cutoff = #{cumsum(sorted_p) <= top_p}`` (ties at the threshold kept),
  then Gumbel-max at the original vocabulary indices.

The top-p rule is evaluated in float64 on exact masses.  Its threshold is the
largest value ``v`` with ``sum(p_i for x_i >= v) > top_p`` -- the same set
``cumsum <= top_p`` selects for any order of equal values.  A row whose
cumulative mass lies within ``MASS_TOL`` of ``top_p`` at the threshold is
reported ambiguous, with both admissible token ids.

Pinned by: tests/test_oracle.py -- brute force over tiny rows (explicit sort +
cumsum exactly as spec_decode.py:72-76 writes it), the invariants
kept >= argmax, |kept| >= min(k, V), mass(kept) > top_p, numpy/torch bf16
rounding, and a float64 dot for the logits.
"""
from __future__ import annotations

import numpy as np

from .jax_random import argmax_first, gumbel

MASS_TOL = 1e-5
# largest / smallest Gumbel draws: u = 1 - 2**-23 and u = tiny
GUMBEL_MAX = np.float32(-np.log(-np.log(np.float64(np.float32(1 - 2.0**-23)))))
GUMBEL_MIN = np.float32(-np.log(-np.log(np.float64(np.finfo(np.float32).tiny))))


# ----------------------------------------------------------------------------- dtypes

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (NaN stays NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    with np.errstate(over="ignore"):
        r = (u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    r = np.where(nan, (u >> np.uint32(16)) | np.uint32(0x40), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


# ----------------------------------------------------------------------------- LM head

def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """layers.py:22-29, in float32 steps."""
    xf = np.asarray(x, dtype=np.float32)
    ms = np.mean(np.square(xf), axis=-1, keepdims=True, dtype=np.float32)
    xn = xf * (np.float32(1.0) / np.sqrt(ms + np.float32(eps), dtype=np.float32))
    return (xn * (np.float32(1.0) + np.asarray(weight, np.float32))).astype(np.float32)


def lm_head_input(hidden: np.ndarray, norm_weight: np.ndarray | None, eps: float = 1e-6, *,
                  hidden_dtype: str = "f32", act_dtype: str = "f32") -> np.ndarray:
    """The LM-head operand of _lm_head_normed_hidden_and_weight (model.py:734-762).

    ``norm_weight`` None: hidden is already normed (``hidden_is_normed=True``).
    Otherwise rms_norm (layers.py:11-29) in float32 steps, its
    ``astype(input_dtype)`` (``hidden_dtype``: "f32" / "bf16" / "f16"), then
    the activation cast (model.py:758-760, ``act_dtype``).  Returns float32."""
    rnd = {"f32": lambda v: np.asarray(v, np.float32), "bf16": round_bf16, "f16": round_f16}
    x = np.asarray(hidden, np.float32)
    if norm_weight is not None:
        x = rnd[hidden_dtype](rms_norm(x, norm_weight, eps))
    return rnd[act_dtype](x)


def lm_head_logits(hidden: np.ndarray, weight: np.ndarray, *, weight_layout: str = "vh") -> np.ndarray:
    """Exact (float64) logits of ``hidden[B,H] . W``.

    ``weight_layout`` "vh" is the tied-embedding storage ``[V, H]``; "hv" is
    the reference's ``lm_head`` / ``embed_tokens.T`` operand ``[H, V]``."""
    h = np.asarray(hidden, dtype=np.float64)
    w = np.asarray(weight, dtype=np.float64)
    if weight_layout == "vh":
        return h @ w.T
    if weight_layout == "hv":
        return h @ w
    raise ValueError(weight_layout)


def greedy_top1(logits64: np.ndarray, reduce_cast: int = 0):
    """Greedy ids from exact logits plus an ambiguity report.

    The kernel accumulates in fp32 (order differs from any other fp32 dot), so
    a row is *ambiguous* when its top-2 gap is below 1e-3 relative -- the
    north-star exemption -- or, with ``reduce_cast``, when a near-maximal
    logit sits within fp32 accumulation error of a bf16/f16 rounding
    boundary.  For ambiguous rows ``admissible[b]`` lists every id a correct
    fp32 kernel may return.

    Returns (ids int64[B], ambiguous bool[B], admissible list[set]).
    """
    z = np.asarray(logits64, dtype=np.float64)
    B, V = z.shape
    ids = np.zeros(B, dtype=np.int64)
    amb = np.zeros(B, dtype=bool)
    adm = []
    for b in range(B):
        row = z[b]
        if reduce_cast:
            rnd = round_bf16 if reduce_cast == 1 else round_f16
            r = rnd(row.astype(np.float32)).astype(np.float64)
        else:
            r = row.astype(np.float32).astype(np.float64)
        ids[b] = int(argmax_first(r))
        top = r[ids[b]]
        scale = max(abs(top), 1e-30)
        # candidates: exact value within 1e-3 relative of the best exact value
        best_exact = np.max(row)
        cand = np.nonzero(row >= best_exact - 1e-3 * max(abs(best_exact), 1e-30))[0]
        if reduce_cast:
            # any logit whose rounded value can reach the rounded maximum
            ulp = np.abs(top) * (2.0 ** -7 if reduce_cast == 1 else 2.0 ** -10)
            cand = np.union1d(cand, np.nonzero(row >= top - ulp)[0])
        srt = np.sort(r)[::-1]
        gap = (srt[0] - srt[1]) / scale if V > 1 else np.inf
        if len(cand) > 1 or gap < 1e-3:
            amb[b] = True
            adm.append(set(int(c) for c in cand) | {int(ids[b])})
        else:
            adm.append({int(ids[b])})
    return ids, amb, adm


# ----------------------------------------------------------------------------- sampler

def scale_logits(l: np.ndarray, temperature: float) -> np.ndarray:
    """``logit / jnp.maximum(T, 1e-6)`` in float32 (model.py:932); NaN propagates."""
    t = np.float32(temperature)
    tp = t if np.isnan(t) else np.maximum(t, np.float32(1e-6))
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        return (np.asarray(l, dtype=np.float32) / tp).astype(np.float32)


def topk_threshold(x: np.ndarray, k: int) -> np.float32:
    """k-th largest value, counting multiplicity."""
    return np.sort(x)[::-1][k - 1]


def topp_threshold(xk: np.ndarray, top_p: float):
    """Top-p threshold over the survivor values ``xk`` (float32).

    Returns (tau, ambiguous, tau_alt): tau is the largest value v with
    mass(x >= v) > top_p * mass(all); ``tau_alt`` is the neighbouring value
    that a fp32 evaluation within MASS_TOL could select instead (or None)."""
    m = np.float64(np.max(xk))
    vals, counts = np.unique(xk.astype(np.float64), return_counts=True)
    vals = vals[::-1]
    counts = counts[::-1]
    e = np.exp(vals - m) * counts
    Z = e.sum()
    cum = np.cumsum(e) / Z  # mass(x >= vals[j])
    p = float(top_p)
    j = int(np.searchsorted(cum, p, side="right"))  # first j with cum[j] > p
    if j >= len(vals):
        j = len(vals) - 1
    tau = vals[j]
    amb = False
    alt = None
    if abs(cum[j] - p) < MASS_TOL and j + 1 < len(vals):
        amb, alt = True, vals[j + 1]
    if j > 0 and abs(cum[j - 1] - p) < MASS_TOL:
        amb, alt = True, vals[j - 1]
    return np.float32(tau), amb, (None if alt is None else np.float32(alt))


def sample_row(l: np.ndarray, temperature: float, top_k: int, top_p: float, key,
               noise: np.ndarray | None = None):
    """Token id for one row plus diagnostics.

    ``noise`` overrides the Gumbel draws (the "identical uniform draws" test
    mode); by default they come from ``gumbel(key, V)``.

    Returns dict(id, ambiguous, ids (admissible set), kept, tau)."""
    l = np.asarray(l, dtype=np.float32)
    V = l.shape[0]
    t = np.float32(temperature)
    if t <= 0:
        i = int(argmax_first(l))
        return dict(id=i, ambiguous=False, ids={i}, kept=None, tau=None)
    x = scale_logits(l, t)
    use_k = 0 < int(top_k) < V
    use_p = float(top_p) < 1.0
    g = gumbel(key, V) if noise is None else np.asarray(noise, np.float32)
    if not (use_k or use_p):
        i = int(argmax_first((x + g).astype(np.float32)))
        return dict(id=i, ambiguous=False, ids={i}, kept=V, tau=None)
    # non-finite rows: the first NaN, else the first +inf, else (all -inf) index 0
    if np.isnan(x).any() or not np.isfinite(np.max(x)):
        i = int(argmax_first(x))
        return dict(id=i, ambiguous=False, ids={i}, kept=None, tau=None)
    thr = topk_threshold(x, int(top_k)) if use_k else np.float32(-np.inf)
    taus = [thr]
    amb = False
    if use_p:
        xk = x[x >= thr]
        tau, amb, alt = topp_threshold(xk, top_p)
        taus = [tau] + ([alt] if amb else [])
    ids = set()
    kept = None
    for n, tau in enumerate(taus):
        keep = x >= tau
        s = np.where(keep, (x + g).astype(np.float32), np.float32(-np.inf))
        ids.add(int(argmax_first(s)))
        if n == 0:
            kept = int(keep.sum())
            first = int(argmax_first(s))
    return dict(id=first, ambiguous=amb and len(ids) > 1, ids=ids, kept=kept, tau=taus[0])


def sample_rows(logits: np.ndarray, temperature, top_k, top_p, keys, noise=None):
    """Row-wise ``sample_row``; returns (ids int64[B], list of per-row dicts)."""
    logits = np.asarray(logits, dtype=np.float32)
    B = logits.shape[0]
    out = np.zeros(B, dtype=np.int64)
    info = []
    for b in range(B):
        key = (np.uint32(keys[b][0]), np.uint32(keys[b][1]))
        r = sample_row(logits[b], temperature[b], top_k[b], top_p[b], key,
                       None if noise is None else noise[b])
        out[b] = r["id"]
        info.append(r)
    return out, info


def order_key(x: np.ndarray) -> np.ndarray:
    """Total-order key of float32 values as used by the library's argmax and
    top-k: larger value -> larger key; every NaN above +inf; -0.0 == +0.0."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).copy()
    u[np.isnan(np.asarray(x, np.float32))] = 0x7FFFFFFF
    u[u == 0x80000000] = 0
    neg = (u & 0x80000000) != 0
    return np.where(neg, ~u, u | np.uint32(0x80000000)).astype(np.uint64)


def topk(logits: np.ndarray, k: int):
    """jax.lax.top_k(logits.astype(float32), k) (model.py:896) per row: values
    (the elements themselves) and int32 indices by value descending, then
    index ascending, with order_key's NaN / signed-zero conventions."""
    x = np.atleast_2d(np.asarray(logits, np.float32))
    vals = np.empty((x.shape[0], k), np.float32)
    idx = np.empty((x.shape[0], k), np.int32)
    for b in range(x.shape[0]):
        key = order_key(x[b])
        order = np.lexsort((np.arange(x.shape[1]), -key.astype(np.int64)))[:k]
        idx[b] = order
        vals[b] = x[b][order]
    return vals, idx
