"""Pins the CPU oracle before it is trusted as the checker (CPU only).

Each check is chosen so that a plausible slip in the restatement -- a wrong
rotation or key-injection, a dropped minus sign in the Gumbel transform, a
reversed tie rule, a cumsum that stops one element early -- fails it.
"""
import math

import numpy as np
import pytest

from oracle import jax_random as jr
from oracle import selection as sel

# Random123 known-answer vectors for threefry2x32_20 (Salmon et al., SC'11;
# kat_vectors in the Random123 distribution).
KAT = [
    ((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
]


@pytest.mark.parametrize("key,ctr,expect", KAT)
def test_threefry_known_answers(key, ctr, expect):
    o0, o1 = jr.threefry2x32((np.uint32(key[0]), np.uint32(key[1])), np.uint32(ctr[0]), np.uint32(ctr[1]))
    assert (int(o0), int(o1)) == expect


def test_threefry_vectorised_matches_scalar():
    key = (np.uint32(0x13198A2E), np.uint32(0x03707344))
    c = np.arange(100, dtype=np.uint32)
    v0, v1 = jr.threefry2x32(key, np.zeros_like(c), c)
    for i in (0, 1, 57, 99):
        s0, s1 = jr.threefry2x32(key, np.uint32(0), np.uint32(i))
        assert (int(v0[i]), int(v1[i])) == (int(s0), int(s1))


def test_prng_key_and_fold_in_structure():
    assert tuple(int(x) for x in jr.prng_key(0)) == (0, 0)
    assert tuple(int(x) for x in jr.prng_key(42)) == (0, 42)
    # fold_in(k, d) is threefry(k, (0, d)); PRNGKey(0) folded with 0 is the first KAT.
    assert tuple(int(x) for x in jr.fold_in(jr.prng_key(0), 0)) == (0x6B200159, 0x99BA4EFE)
    # partitionable split uses the flat index as the counter: split(k)[0] == threefry(k,(0,0))
    s = jr.split(jr.prng_key(0), 2)
    assert tuple(int(x) for x in s[0]) == (0x6B200159, 0x99BA4EFE)
    assert tuple(int(x) for x in s[1]) == tuple(int(x) for x in jr.fold_in(jr.prng_key(0), 1))


def test_random_bits_counter_layout_crosses_32_bits():
    key = jr.prng_key(3)
    start = 2**32 - 2
    bits = jr.random_bits32(key, 4, start=start)
    for j in range(4):
        i = start + j
        o0, o1 = jr.threefry2x32(key, np.uint32(i >> 32), np.uint32(i & 0xFFFFFFFF))
        assert int(bits[j]) == int(o0 ^ o1)


def test_uniform_and_gumbel_extremes():
    bits = np.array([0, 0x1FF, 0x200, 0xFFFFFFFF], dtype=np.uint32)
    u = jr.uniform_from_bits(bits, jr.TINY_F32, np.float32(1.0))
    assert u[0] == jr.TINY_F32 and u[1] == jr.TINY_F32  # the low 9 bits are discarded
    assert u[2] == np.float32(2.0**-23)
    assert u[3] == np.float32(1.0 - 2.0**-23)
    g = jr.gumbel_from_bits(bits)
    assert g[0] == sel.GUMBEL_MIN and g[3] == sel.GUMBEL_MAX
    assert abs(float(g[0]) - (-math.log(-math.log(np.finfo(np.float32).tiny)))) < 1e-5
    assert np.all(np.diff(g[[0, 2, 3]]) > 0)  # monotone in the draw


def test_gumbel_moments():
    g = jr.gumbel(jr.prng_key(11), 400_000).astype(np.float64)
    euler = 0.5772156649
    assert abs(g.mean() - euler) < 0.01
    assert abs(g.var() - math.pi**2 / 6) < 0.02


def test_categorical_frequencies_follow_softmax():
    logits = np.array([0.3, -1.2, 1.5, 0.0, 0.9], dtype=np.float32)
    n = 40_000
    base = jr.prng_key(5)
    counts = np.zeros(5)
    # one draw per key, keys from fold_in as the executor derives them
    for c in range(n):
        counts[jr.categorical(jr.fold_in(base, c), logits)] += 1
    p = np.exp(logits - logits.max())
    p /= p.sum()
    chi2 = float(((counts - n * p) ** 2 / (n * p)).sum())
    assert chi2 < 25.0, (counts / n, p)  # 4 dof; 25 is far in the tail


def test_argmax_first_semantics():
    assert jr.argmax_first(np.array([1.0, 3.0, 3.0, 2.0], np.float32)) == 1
    assert jr.argmax_first(np.array([1.0, np.nan, 5.0, np.nan], np.float32)) == 1
    assert jr.argmax_first(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert jr.argmax_first(np.array([-0.0, 0.0], np.float32)) == 0


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.00390625, 1.01171875, np.inf, -np.inf, 3.4e38], np.float32)])
    ours = sel.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def _brute_topp_keep(x, top_p):
    """spec_decode.py:71-76 written out literally, in float64."""
    p = np.exp(x.astype(np.float64) - x.max())
    p /= p.sum()
    sp = np.sort(p)[::-1]
    cs = np.cumsum(sp)
    cut = int(np.sum(cs <= top_p))
    cut = min(cut, len(sp) - 1)  # jnp gather clamps
    return p >= sp[cut]


def test_topp_threshold_matches_literal_formula():
    rng = np.random.default_rng(1)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(2, 40))
        x = (rng.standard_normal(n) * rng.uniform(0.3, 3)).astype(np.float32)
        if trial % 3 == 0:  # force ties
            x = np.round(x * 2) / 2
        top_p = float(rng.uniform(0.05, 0.99))
        tau, amb, _ = sel.topp_threshold(x, top_p)
        if amb:
            continue
        keep = x >= tau
        assert np.array_equal(keep, _brute_topp_keep(x, top_p)), (x, top_p)
        checked += 1
    assert checked > 250


def test_sample_row_invariants():
    rng = np.random.default_rng(2)
    V = 3000
    for trial in range(20):
        l = (rng.standard_normal(V) * 3).astype(np.float32)
        k = int(rng.choice([0, 1, 5, 50]))
        p = float(rng.choice([1.0, 0.9, 0.5]))
        key = jr.fold_in(jr.prng_key(0), trial)
        r = sel.sample_row(l, 0.8, k, p, key)
        x = sel.scale_logits(l, 0.8)
        if k or p < 1:
            assert r["kept"] >= 1
            if k:
                if p == 1.0:
                    assert r["kept"] >= min(k, V)
                assert x[r["id"]] >= np.sort(x)[::-1][k - 1]
            if k == 0 and p < 1:
                e = np.exp(x.astype(np.float64) - x.max())
                assert e[x >= r["tau"]].sum() / e.sum() > p - 1e-9
            assert x[r["id"]] >= r["tau"]
        # the filtered draw equals categorical over the masked logits
        if k or p < 1:
            masked = np.where(x >= r["tau"], x, np.float32(-np.inf))
            assert r["id"] == jr.categorical(key, masked)
    # greedy rows ignore k / p and the key
    l = np.array([0.5, 2.0, 2.0, -1.0], np.float32)
    assert sel.sample_row(l, 0.0, 2, 0.5, jr.prng_key(0))["id"] == 1


def test_sample_row_temperature_route_is_categorical():
    rng = np.random.default_rng(3)
    l = rng.standard_normal(1000).astype(np.float32)
    key = jr.engine_key(3, 7)
    expect = jr.categorical(key, (l / np.float32(0.7)).astype(np.float32))
    assert sel.sample_row(l, 0.7, 0, 1.0, key)["id"] == expect


def test_sample_row_nonfinite_rows():
    key = jr.prng_key(0)
    l = np.array([1.0, np.nan, 3.0, np.nan], np.float32)
    assert sel.sample_row(l, 1.0, 2, 0.9, key)["id"] == 1
    l = np.array([1.0, np.inf, 3.0, np.inf], np.float32)
    assert sel.sample_row(l, 1.0, 2, 0.9, key)["id"] == 1
    l = np.full(5, -np.inf, np.float32)
    assert sel.sample_row(l, 1.0, 2, 0.9, key)["id"] == 0


def test_greedy_top1_oracle_against_float64_dot():
    rng = np.random.default_rng(4)
    h = rng.standard_normal((5, 64)).astype(np.float32)
    w = (rng.standard_normal((300, 64)) * 0.02).astype(np.float32)
    z = sel.lm_head_logits(h, w, weight_layout="vh")
    assert np.allclose(z, h.astype(np.float64) @ w.astype(np.float64).T)
    assert np.allclose(sel.lm_head_logits(h, w.T.copy(), weight_layout="hv"), z)
    ids, amb, adm = sel.greedy_top1(z)
    assert np.array_equal(ids, np.argmax(z, axis=1))
    for b in range(5):
        assert ids[b] in adm[b]


def test_rms_norm_formula():
    x = np.array([[3.0, 4.0]], np.float32)
    w = np.array([0.0, 1.0], np.float32)
    out = sel.rms_norm(x, w, eps=0.0)
    rms = math.sqrt((9 + 16) / 2)
    assert np.allclose(out, [[3 / rms, 2 * 4 / rms]], rtol=1e-6)


def test_lm_head_input_pins():
    """The pre-norm LM-head operand: closed forms, torch's RMSNorm, rounding order."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    # constant rows normalise to +-1 whatever their scale (eps = 0, w = 0)
    x = np.array([[3.0] * 8, [-0.25] * 8], np.float32)
    out = sel.lm_head_input(x, np.zeros(8, np.float32), 0.0)
    assert np.array_equal(out, np.array([[1.0] * 8, [-1.0] * 8], np.float32))
    # against torch.nn.functional.rms_norm (fp32) times (1 + w)
    x = rng.normal(0, 2.0, (4, 1024)).astype(np.float32)
    w = rng.normal(0, 0.1, 1024).astype(np.float32)
    ref = (torch.nn.functional.rms_norm(torch.from_numpy(x), (1024,), eps=1e-6)
           * (1.0 + torch.from_numpy(w))).numpy()
    got = sel.lm_head_input(x, w, 1e-6)
    assert np.allclose(got, ref, rtol=4e-7 * 4, atol=0)
    # unit mean square after the norm (w = 0)
    got0 = sel.lm_head_input(x, np.zeros(1024, np.float32), 1e-6).astype(np.float64)
    assert np.allclose(np.mean(got0 ** 2, axis=1), 1.0, rtol=1e-5)
    # rounding: to the hidden's own type first, then to the activation type
    xb = sel.round_bf16(x)
    two = sel.lm_head_input(xb, w, 1e-6, hidden_dtype="bf16", act_dtype="f32")
    assert np.array_equal(two, sel.round_bf16(sel.rms_norm(xb, w, 1e-6)))
    act = sel.lm_head_input(x, w, 1e-6, hidden_dtype="f32", act_dtype="bf16")
    assert np.array_equal(act, sel.round_bf16(got))
    # hidden already normed: only the activation cast
    assert np.array_equal(sel.lm_head_input(x, None, act_dtype="bf16"), sel.round_bf16(x))


def test_topk_oracle_pins():
    """Top-k order: textbook stable sort for finite data, torch.topk values,
    argmax agreement (first NaN, -0 == +0), brute force on tiny rows."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = rng.normal(0, 1, (3, 1000)).astype(np.float32)
    x[:, 10] = x[:, 20] = x[:, 900] = 7.0  # ties at the top keep index order
    v, i = sel.topk(x, 17)
    for b in range(3):
        assert np.array_equal(i[b], np.argsort(-x[b], kind="stable")[:17])
    tv, _ = torch.topk(torch.from_numpy(x), 17, sorted=True)
    assert np.array_equal(v, tv.numpy())
    assert np.array_equal(i[:, :3], np.array([[10, 20, 900]] * 3))
    # NaN orders first (the first NaN first), then +inf; signed zeros tie
    y = np.array([1.0, np.nan, -0.0, np.inf, 0.0, np.nan, -np.inf], np.float32)
    v, i = sel.topk(y, 7)
    assert i[0].tolist() == [1, 5, 3, 0, 2, 4, 6]
    assert np.array_equal(v[0].view(np.uint32), y[i[0]].view(np.uint32))
    assert sel.topk(y, 1)[1][0, 0] == jr.argmax_first(y[None])[0]
    assert sel.topk(np.array([[-0.0, 0.0]], np.float32), 1)[1][0, 0] == 0
    # brute force over all permutations of a tiny row with ties
    import itertools
    base = np.array([2.0, -1.0, 2.0, 0.5, -1.0], np.float32)
    for perm in itertools.permutations(range(5)):
        row = base[list(perm)]
        got = sel.topk(row, 3)[1][0].tolist()
        exp = sorted(range(5), key=lambda j: (-row[j], j))[:3]
        assert got == exp
