"""CPU oracle: numpy restatement of the JAX random pieces the sampler uses.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path imports this module;
only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
use it, and only as the checker.

The reference samples with ``jax.random.categorical`` under per-row keys
``fold_in(fold_in(PRNGKey(0), slot), counter)``
(nanovllm_jax/engine/model_executor.py:2131, 2214-2219;
nanovllm_jax/model.py:929-936).  JAX itself (jax/jaxlib 0.6.2, uv.lock:662-700)
is not installed here, so its published algorithm is restated:

* ``threefry2x32`` -- Threefry-2x32 with 20 rounds (Salmon et al., SC'11,
  "Parallel random numbers: as easy as 1, 2, 3"), rotation schedule
  {13,15,26,6} / {17,29,16,24}, key-schedule parity constant 0x1BD11BDA and a
  key injection (with the injection counter added to word 1) after every four
  rounds.
* ``prng_key(seed)``  = (seed >> 32, seed & 0xFFFFFFFF) -> (0, seed) for 32-bit seeds.
* ``fold_in(key, d)`` = threefry2x32(key, (0, d)).
* ``random_bits32(key, n)[i]`` = o0 ^ o1 with (o0, o1) = threefry2x32(key,
  (hi32(i), lo32(i))) -- the partitionable counter layout that is the JAX
  default since 0.5 (``jax_threefry_partitionable``).
* ``uniform``  f = bitcast((bits >> 9) | 0x3F800000) - 1;
  u = max(minval, f * (maxval - minval) + minval).
* ``gumbel`` (mode "low") = -log(-log(uniform(minval=tiny, maxval=1))).
* ``categorical(key, logits)`` = argmax(gumbel(key, logits.shape) + logits).

Each float32 operation is rounded to float32 after it is performed.  ``log``
is evaluated in float64 and rounded once to float32 (a correctly rounded
float32 log); XLA-CPU's own ``log`` ulp behaviour is not available to pin.

Pinned by: Random123 known-answer vectors (tests/test_oracle.py), and the
special cases of the float construction (bits 0 -> tiny, all-ones -> 1-2^-23).
"""
from __future__ import annotations

import numpy as np

U32 = np.uint32
_MASK = 0xFFFFFFFF
_ROT0 = (13, 15, 26, 6)
_ROT1 = (17, 29, 16, 24)
TINY_F32 = np.float32(np.finfo(np.float32).tiny)


def _rotl(v: np.ndarray, r: int) -> np.ndarray:
    return (v << U32(r)) | (v >> U32(32 - r))


def threefry2x32(key, x0, x1):
    """Threefry-2x32-20 over broadcastable uint32 arrays.

    ``key`` is a pair (k0, k1) of uint32 scalars or arrays.  Returns (o0, o1).
    """
    k0 = np.asarray(key[0], dtype=U32)
    k1 = np.asarray(key[1], dtype=U32)
    k2 = k0 ^ k1 ^ U32(0x1BD11BDA)
    ks = (k0, k1, k2)
    with np.errstate(over="ignore"):
        v0 = np.asarray(x0, dtype=U32) + k0
        v1 = np.asarray(x1, dtype=U32) + k1
        for block in range(5):
            rots = _ROT0 if block % 2 == 0 else _ROT1
            for r in rots:
                v0 = v0 + v1
                v1 = _rotl(v1, r)
                v1 = v1 ^ v0
            # key injection s = block + 1
            s = block + 1
            v0 = v0 + ks[s % 3]
            v1 = v1 + ks[(s + 1) % 3] + U32(s)
    return v0.astype(U32), v1.astype(U32)


def prng_key(seed: int):
    """``jax.random.PRNGKey(seed)`` for a non-negative seed below 2**32."""
    seed = int(seed)
    return (U32((seed >> 32) & _MASK), U32(seed & _MASK))


def fold_in(key, data: int):
    """``jax.random.fold_in(key, data)`` = threefry2x32(key, (0, uint32(data)))."""
    o0, o1 = threefry2x32(key, U32(0), U32(int(data) & _MASK))
    return (U32(o0), U32(o1))


def split(key, num: int = 2):
    """Partitionable ``jax.random.split``: key i = threefry2x32(key, (0, i))."""
    i = np.arange(num, dtype=np.uint64)
    o0, o1 = threefry2x32(key, (i >> np.uint64(32)).astype(U32), (i & np.uint64(_MASK)).astype(U32))
    return np.stack([o0, o1], axis=-1)


def engine_key(slot: int, counter: int):
    """Per-row sampling key of the executor's sampled route
    (model_executor.py:2131, 2214-2219): fold_in(fold_in(PRNGKey(0), slot), counter)."""
    return fold_in(fold_in(prng_key(0), slot), counter)


def random_bits32(key, n: int, start: int = 0) -> np.ndarray:
    """Partitionable ``random_bits(key, 32, (n,))`` for flat indices [start, start+n)."""
    i = np.arange(start, start + n, dtype=np.uint64)
    o0, o1 = threefry2x32(key, (i >> np.uint64(32)).astype(U32), (i & np.uint64(_MASK)).astype(U32))
    return o0 ^ o1


def bits_to_unit_float(bits: np.ndarray) -> np.ndarray:
    """JAX's mantissa trick: float in [0, 1) from the top 23 bits."""
    fb = (bits >> U32(9)) | U32(0x3F800000)
    return fb.view(np.float32) - np.float32(1.0)


def uniform_from_bits(bits: np.ndarray, minval=np.float32(0.0), maxval=np.float32(1.0)) -> np.ndarray:
    minval = np.float32(minval)
    maxval = np.float32(maxval)
    f = bits_to_unit_float(bits)
    span = np.float32(maxval - minval)
    return np.maximum(minval, (f * span).astype(np.float32) + minval).astype(np.float32)


def log_f32(x: np.ndarray) -> np.ndarray:
    """float32 log, correctly rounded (float64 evaluation, one rounding)."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.log(np.asarray(x, dtype=np.float64)).astype(np.float32)


def gumbel_from_bits(bits: np.ndarray) -> np.ndarray:
    """``jax.random.gumbel`` (mode "low") given the raw random bits."""
    u = uniform_from_bits(bits, TINY_F32, np.float32(1.0))
    return -log_f32(-log_f32(u))


def gumbel(key, n: int, start: int = 0) -> np.ndarray:
    return gumbel_from_bits(random_bits32(key, n, start))


def argmax_first(x: np.ndarray, axis: int = -1) -> np.ndarray:
    """``jnp.argmax``: index of the first maximum; the first NaN wins.

    numpy's argmax has the same contract (NaN propagates as the maximum and the
    first occurrence is returned)."""
    return np.argmax(x, axis=axis)


def categorical(key, logits: np.ndarray) -> int:
    """``jax.random.categorical(key, logits)`` for a 1-D float32 row."""
    logits = np.asarray(logits, dtype=np.float32)
    g = gumbel(key, logits.shape[0])
    return int(argmax_first((g + logits).astype(np.float32)))
