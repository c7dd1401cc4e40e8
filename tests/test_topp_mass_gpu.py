"""GPU parity: the top-p threshold and the kept softmax mass, directly.

The reference's top-p rule (nanovllm_jax/spec_decode.py:69-83: sort, softmax,
cumsum, keep ``p >= sorted_p[#{cumsum <= top_p}]``, ties kept) is evaluated by
the kernels in fixed point (top-k survivors) or on a 1/32-nat grid of bins
(top-p-only rows).  ``nvjsel_debug_sample_topp`` reports, per row, the
threshold tau the kernels settled on and the mass of the kept set over the
top-k survivors as the kernels computed it.  Against the float64 oracle:

* tau must equal the oracle's threshold bit for bit, except on rows the oracle
  reports as mass-ambiguous (cumulative mass within 1e-5 of top_p at the
  threshold), where it may be the neighbouring value -- such rows are printed;
* |kernel mass - float64 mass of the same kept set| <= 1e-5 on every row
  (the north star's "intermediate fp32 softmax mass within 1e-5").
"""
import ctypes

import numpy as np
import pytest
import torch

import nvjsel
from nvjsel import _lib
from oracle import selection as sel
from tests.gpu_helpers import keys_tensor, report

pytestmark = pytest.mark.gpu

MASS_TOL = 1e-5


def _debug_sample(logits: torch.Tensor, temps, top_k, top_p, keys_i32: torch.Tensor):
    B, V = logits.shape
    dt = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}[logits.dtype]
    dev = logits.device
    t = torch.as_tensor(temps, dtype=torch.float32, device=dev).contiguous()
    k = torch.as_tensor(top_k, dtype=torch.int32, device=dev).contiguous()
    p = torch.as_tensor(top_p, dtype=torch.float32, device=dev).contiguous()
    ids = torch.empty(B, dtype=torch.int32, device=dev)
    tau = torch.empty(B, dtype=torch.float32, device=dev)
    mass = torch.empty(B, dtype=torch.float64, device=dev)
    lib = _lib.load()
    nbytes = lib.nvjsel_sample_workspace_size(B, V)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=dev)  # zero at rest (include/nvjsel.h)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    _lib.call("nvjsel_debug_sample_topp", logits.data_ptr(), dt, B, V, nvjsel.selection._row_stride(logits), t.data_ptr(),
              k.data_ptr(), p.data_ptr(), keys_i32.data_ptr(), ids.data_ptr(), tau.data_ptr(), mass.data_ptr(),
              ws.data_ptr(), nbytes, stream)
    torch.cuda.synchronize()
    return ids.cpu().numpy(), tau.cpu().numpy(), mass.cpu().numpy()


def _oracle_row(l, T, k, p):
    """(tau, mass at tau, ambiguous, alternative tau, mass at the alternative)
    or None for rows without a threshold (greedy, unfiltered, non-finite)."""
    if T <= 0:
        return None
    x = sel.scale_logits(l, T)
    V = x.shape[0]
    use_k, use_p = 0 < k < V, p < 1.0
    if not (use_k or use_p) or not np.isfinite(x).all():
        return None
    thr = sel.topk_threshold(x, k) if use_k else np.float32(-np.inf)
    xk = x[x >= thr].astype(np.float64)
    w = np.exp(xk - xk.max())
    Z = w.sum()

    def mass(t):
        return float(w[xk >= float(t)].sum() / Z)

    if not use_p:
        return thr, 1.0, False, None, None
    tau, amb, alt = sel.topp_threshold(x[x >= thr], p)
    return tau, mass(tau), amb, alt, (None if alt is None else mass(alt))


def _check(name, logits: torch.Tensor, T, K, P, keys_i32):
    ids, tau, mass = _debug_sample(logits, T, K, P, keys_i32)
    # the debug entry's ids are the plain entry's
    plain = nvjsel.sample_token_ids(logits, torch.as_tensor(T, device=logits.device), keys_i32,
                                    top_k=torch.as_tensor(K, dtype=torch.int32, device=logits.device),
                                    top_p=torch.as_tensor(P, dtype=torch.float32, device=logits.device))
    assert np.array_equal(ids, plain.cpu().numpy())
    used = logits.float().cpu().numpy()
    worst, n_rows, exempt = 0.0, 0, []
    for b in range(used.shape[0]):
        o = _oracle_row(used[b], float(T[b]), int(K[b]), float(P[b]))
        if o is None:
            assert np.isnan(tau[b]) and np.isnan(mass[b]), f"{name} row {b}: threshold reported on an unfiltered row"
            continue
        t_o, m_o, amb, alt, m_alt = o
        n_rows += 1
        if np.float32(tau[b]).view(np.uint32) == np.float32(t_o).view(np.uint32):
            ref = m_o
        else:
            assert amb and alt is not None and np.float32(tau[b]) == np.float32(alt), (
                f"{name} row {b}: tau {tau[b]!r} vs oracle {t_o!r} (T={T[b]}, k={K[b]}, p={P[b]})")
            exempt.append((b, float(m_o) - float(P[b])))
            ref = m_alt
        err = abs(float(mass[b]) - ref)
        worst = max(worst, err)
        assert err <= MASS_TOL, f"{name} row {b}: kept mass {mass[b]:.9f} vs float64 {ref:.9f}"
        # the kept set's mass exceeds top_p (spec_decode.py:72-76 keeps the crossing element)
        if P[b] < 1.0 and not amb:
            assert mass[b] > float(P[b]) - MASS_TOL
    report(f"{name}: {n_rows} thresholded rows, worst |mass - float64| = {worst:.3e}; "
           f"ambiguity-exempt rows (row, oracle mass - p): {exempt}")
    return n_rows, exempt


def _bench_inputs(name):
    import bench

    return bench.make_inputs(torch, name, torch.device("cuda:0"))


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_topp_threshold_and_mass_on_bench_workloads(name):
    """C3 [64, 248320] f32 (k=50, p=0.9, T=0.8) and C5 [256, 248320] bf16
    (mixed per-row T / k / p): every thresholded row's tau and kept mass."""
    d = _bench_inputs(name)
    B = d["batch"]
    print(f"case {name} B={B}", flush=True)
    T = d["temperature"].cpu().numpy()
    K = d["top_k"].cpu().numpy()
    P = d["top_p"].cpu().numpy()
    n_rows, exempt = _check(name, d["logits"], T, K, P, d["keys"])
    assert n_rows > 0
    assert len(exempt) <= max(1, B // 16)


def test_topp_only_rows_and_slow_paths():
    """Top-p-only rows (grid-bin histograms), k > 256 (whole-row radix
    descent) and top-k-only rows, f32 and bf16."""
    rng = np.random.default_rng(11)
    B, V = 12, 100_003
    l = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    T = np.array([1.0, 0.7, 1.3, 1.0, 0.5, 1.0, 0.9, 1.0, 2.0, 1.0, 0.8, 1.0], np.float32)
    K = np.array([0, 0, 0, 300, 1000, 20, 0, 5, 0, 2000, 100, 0], np.int32)
    P = np.array([0.9, 0.5, 0.99, 0.9, 0.8, 1.0, 0.3, 1.0, 0.95, 0.6, 0.95, 0.999], np.float32)
    keys = keys_tensor(np.stack([np.array([b, 7 * b + 1], np.uint32) for b in range(B)]))
    for dt in (torch.float32, torch.bfloat16):
        lt = torch.from_numpy(l).cuda().to(dt)
        _check(f"mixed-{dt}", lt, T, K, P, keys)


@pytest.mark.parametrize("offset", [2e-5, -2e-5, 3e-6, -3e-6, 0.0])
def test_topp_target_near_a_bin_edge(offset):
    """Top-p-only row whose cumulative mass at a grid-bin edge is top_p +
    offset: one level of values per 1/32-nat bin, so the threshold is one of
    two values.  The chunk histograms carry weights in 2^-17 units (a row's
    sums within 4e-6 relative of the 2^-40 ones); 2e-5 away from the edge
    the kernel must pick the oracle's threshold, closer it may pick either,
    and the kept mass stays within 1e-5 either way."""
    V = 65_536
    rng = np.random.default_rng(12)
    levels = np.array([0.0, -1.0, -2.0, -3.0], np.float32)
    counts = np.array([900, 3000, 12000, V - 15900])
    row = np.repeat(levels, counts)[rng.permutation(V)].astype(np.float32)
    w = np.exp(levels.astype(np.float64)) * counts
    cum1 = w[0] / w.sum()  # mass(x >= 0)
    p = np.float32(cum1 - offset)
    o = _oracle_row(row, 1.0, 0, float(p))
    lt = torch.from_numpy(np.ascontiguousarray(row[None, :])).cuda()
    keys = keys_tensor(np.array([[3, 4]], np.uint32))
    ids, tau, mass = _debug_sample(lt, [1.0], [0], [float(p)], keys)
    print(f"offset {offset}: p={float(p):.9f} tau={tau[0]} mass={mass[0]:.9f} oracle tau={o[0]} "
          f"mass={o[1]:.9f} ambiguous={o[2]}", flush=True)
    if abs(offset) >= 1e-5:
        assert not o[2]
    _check(f"edge{offset}", lt, [1.0], [0], [float(p)], keys)
