"""GPU parity: the logits sampler and key derivation (libnvjsel) against the oracle.

The temperature route mirrors the reference's only sampler test
(tests/test_lm_head_helpers.py:218-262: T=[0, 0.7], ids equal
[argmax(l0), categorical(k1, l1/0.7)]); top-k / top-p follow the build's spec
(the reference has no serving top-k/top-p sampler)."""
import numpy as np
import pytest
import torch

import nvjsel
from oracle import jax_random as jr
from oracle import selection as sel
from tests.gpu_helpers import check_sampled, engine_keys, keys_tensor, zipf_logits

pytestmark = pytest.mark.gpu


def _sample(logits_np, temps, top_k=None, top_p=None, keys=None, dtype=torch.float32, noise=None):
    B, V = logits_np.shape
    keys = engine_keys(B) if keys is None else keys
    lt = torch.from_numpy(logits_np).to(dtype).cuda()
    out = nvjsel.sample_token_ids(
        lt, torch.tensor(temps, dtype=torch.float32).cuda(), keys_tensor(keys),
        top_k=None if top_k is None else torch.tensor(top_k, dtype=torch.int32).cuda(),
        top_p=None if top_p is None else torch.tensor(top_p, dtype=torch.float32).cuda(),
        noise=None if noise is None else torch.from_numpy(noise).cuda())
    torch.cuda.synchronize()
    used = lt.float().cpu().numpy()  # the values the kernel saw (bf16-rounded if bf16)
    return out.cpu().numpy(), used, keys


def test_reference_sampler_case_greedy_and_temperature():
    rng = np.random.default_rng(7)
    l = rng.standard_normal((2, 7)).astype(np.float32)
    keys = jr.split(jr.prng_key(7), 2)
    ids, used, _ = _sample(l, [0.0, 0.7], keys=keys)
    assert ids[0] == np.argmax(l[0])
    assert ids[1] == jr.categorical((keys[1, 0], keys[1, 1]), (l[1] / np.float32(0.7)).astype(np.float32))


def test_temperature_full_vocab_c2():
    """f32 [8, 248320] ~N(0,3) + 5 spikes/row at +12, T=0.7, seed=row."""
    rng = np.random.default_rng(1)
    B, V = 8, 248320
    l = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    for b in range(B):
        l[b, rng.choice(V, 5, replace=False)] += 12.0
    keys = np.stack([np.array([int(x) for x in jr.prng_key(b)], np.uint32) for b in range(B)])
    ids, used, _ = _sample(l, [0.7] * B, keys=keys)
    check_sampled(ids, used, [0.7] * B, [0] * B, [1.0] * B, keys, ctx="C2")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_greedy_rows_all_dtypes(dtype):
    rng = np.random.default_rng(2)
    l = rng.standard_normal((5, 30011)).astype(np.float32)
    l[3, 100] = l[3, 29000] = 50.0  # tie: lowest index
    ids, used, _ = _sample(l, [0.0, -1.0, 0.0, 0.0, 0.0], top_k=[5] * 5, top_p=[0.5] * 5, dtype=dtype)
    assert np.array_equal(ids, np.argmax(used, axis=1))
    assert ids[3] == 100


def test_topk_topp_c3_shape():
    """BASELINE config 2 (at B=8): log Zipf(1.1) permuted + N(0,0.5), k=50, p=0.9, T=0.8."""
    rng = np.random.default_rng(3)
    B, V = 8, 248320
    l = zipf_logits(rng, B, V, 1.1, 1.1, 0.5)
    ids, used, keys = _sample(l, [0.8] * B, top_k=[50] * B, top_p=[0.9] * B)
    check_sampled(ids, used, [0.8] * B, [50] * B, [0.9] * B, keys, ctx="C3")


def test_mixed_rows_c5_shape_bf16():
    """BASELINE config 4 (at B=24): bf16 Zipf(1.05..1.3) + N(0,1), mixed T/k/p per row."""
    rng = np.random.default_rng(4)
    B, V = 24, 248320
    l = zipf_logits(rng, B, V, 1.05, 1.3, 1.0)
    T = [float(x) for x in rng.choice([0.0, 0.6, 1.0], B)]
    K = [int(x) for x in rng.choice([0, 20, 100], B)]
    P = [float(x) for x in rng.choice([1.0, 0.95, 0.8], B)]
    ids, used, keys = _sample(l, T, top_k=K, top_p=P, dtype=torch.bfloat16)
    check_sampled(ids, used, T, K, P, keys, ctx="C5")


@pytest.mark.parametrize("k,p", [(1, 1.0), (2, 1.0), (7, 0.5), (0, 0.3), (0, 0.999), (0, 0.0),
                                 (4999, 1.0), (5000, 1.0), (6000, 0.9), (-1, 0.7)])
def test_filter_parameter_edges(k, p):
    rng = np.random.default_rng(5)
    B, V = 6, 5000
    l = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    T = [0.9] * B
    ids, used, keys = _sample(l, T, top_k=[k] * B, top_p=[p] * B)
    check_sampled(ids, used, T, [k] * B, [p] * B, keys, ctx=f"k={k},p={p}")


def test_heavy_ties_and_quantised_logits():
    rng = np.random.default_rng(6)
    B, V = 6, 20000
    l = np.round(rng.standard_normal((B, V)) * 2).astype(np.float32)  # ~9 distinct values
    l[5] = 1.0  # constant row
    T = [1.0] * B
    K = [3, 100, 0, 0, 50, 10]
    P = [1.0, 0.9, 0.5, 0.95, 0.7, 0.5]
    ids, used, keys = _sample(l, T, top_k=K, top_p=P)
    check_sampled(ids, used, T, K, P, keys, ctx="ties")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_onepass_matches_pipeline(dtype):
    """Calls without top-k/top-p arrays take the one-pass Gumbel-max; the same
    rows passed with disabled arrays (k=0, p=1) take the scan/select/gumbel
    pipeline.  Both are exact, so the ids must agree row for row; the oracle
    pins them too.  Rows: greedy, several temperatures, spikes, a NaN row, a
    +inf row, an all -inf row."""
    B, V = 12, 50_021
    rng = np.random.default_rng(321)
    l = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    l[2, rng.choice(V, 5, replace=False)] += 12.0
    l[5, [777, 40_000]] = np.nan
    l[6, [9_000, 30_000]] = np.inf
    l[7] = -np.inf
    T = [0.0, 0.7, 1.0, 0.3, 2.0, 1.0, 1.0, 1.0, 0.0, 0.05, 1.0, 0.7]
    keys = engine_keys(B, 5)
    ids1, used, _ = _sample(l, T, keys=keys, dtype=dtype)
    ids2, _, _ = _sample(l, T, top_k=[0] * B, top_p=[1.0] * B, keys=keys, dtype=dtype)
    assert ids1.tolist() == ids2.tolist()
    assert ids1[5] == 777 and ids1[6] == 9_000 and ids1[7] == 0
    check_sampled(ids1, used, T, [0] * B, [1.0] * B, keys, ctx="onepass")


def test_nonfinite_rows():
    B, V = 5, 4000
    rng = np.random.default_rng(7)
    l = rng.standard_normal((B, V)).astype(np.float32)
    l[0, [10, 20]] = np.nan
    l[1, [30, 3000]] = np.inf
    l[2] = -np.inf
    l[3, :] = -np.inf
    l[3, 1234] = 2.0  # one finite value
    l[4, 5] = -np.inf
    T = [1.0] * B
    ids, used, keys = _sample(l, T, top_k=[5] * B, top_p=[0.9] * B)
    assert ids[0] == 10 and ids[1] == 30 and ids[2] == 0 and ids[3] == 1234
    check_sampled(ids, used, T, [5] * B, [0.9] * B, keys, ctx="nonfinite")
    # unfiltered temperature rows follow categorical (NaN first, +inf first)
    ids2, used2, keys2 = _sample(l[:2], [1.0, 1.0])
    assert ids2[0] == 10 and ids2[1] == 30


def test_external_noise_mode():
    """Identical draws: ids equal argmax over kept of x + noise exactly."""
    rng = np.random.default_rng(8)
    B, V = 4, 10000
    l = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    noise = rng.gumbel(size=(B, V)).astype(np.float32)
    T, K, P = [0.7, 1.0, 1.3, 0.5], [0, 10, 0, 200], [1.0, 1.0, 0.8, 0.9]
    ids, used, keys = _sample(l, T, top_k=K, top_p=P, noise=noise)
    check_sampled(ids, used, T, K, P, keys, noise=noise, ctx="noise")


def test_real_logits_row_fixture():
    """The reference's real Qwen3.5-0.8B logits row (results/qwen08_hf_logits_serving_workloads.npz)."""
    import os
    path = os.path.join(os.path.dirname(__file__), "golden", "qwen08_logits_row.npz")
    row = np.load(path)["logits_0"].astype(np.float32)
    assert int(np.argmax(row)) == 13
    l = np.stack([row] * 6)
    T = [0.0, 0.7, 1.0, 1.0, 0.6, 1.2]
    K = [0, 0, 50, 0, 20, 1000]
    P = [1.0, 1.0, 0.9, 0.95, 0.8, 0.99]
    ids, used, keys = _sample(l, T, top_k=K, top_p=P)
    assert ids[0] == 13
    check_sampled(ids, used, T, K, P, keys, ctx="qwen-row")


def test_derive_keys_matches_fold_in_chain():
    slots = np.array([0, 1, 5, 1000, -3, 7], np.int32)
    counters = np.array([0, 0, 17, 2**31 - 1, 4, -1], np.int32)
    keys, nxt = nvjsel.derive_rng_keys(torch.from_numpy(slots).cuda(), torch.from_numpy(counters).cuda())
    torch.cuda.synchronize()
    got = keys.cpu().numpy().view(np.uint32)
    for b in range(len(slots)):
        exp = jr.engine_key(max(0, int(slots[b])), int(counters[b]) & 0xFFFFFFFF)
        assert tuple(int(x) for x in got[b]) == (int(exp[0]), int(exp[1]))
    assert np.array_equal(nxt.cpu().numpy(), (counters.astype(np.int64) + 1).astype(np.int32))


def test_counter_table_keys_and_bump():
    """Device-resident counters (model_executor.py:3593-3619): gather, fold_in
    chain, table.at[slots].set(counter + 1); negative slots use slot 0, slots
    past the table read its last entry and are not written."""
    table = torch.zeros(16, dtype=torch.int32).cuda()
    table[15] = 9
    slots = np.array([3, 5, -1, 3, 20, 15], np.int32)
    st = torch.from_numpy(slots).cuda()
    for step in range(3):
        before = table.cpu().numpy().copy()
        keys = nvjsel.derive_rng_keys_from_table(st, table)
        torch.cuda.synchronize()
        got = keys.cpu().numpy().view(np.uint32)
        for b, slot in enumerate(slots):
            s_eff = max(0, int(slot))
            ctr = int(before[min(s_eff, 15)])
            exp = jr.engine_key(s_eff, ctr)
            assert tuple(int(x) for x in got[b]) == (int(exp[0]), int(exp[1])), (step, b)
        after = table.cpu().numpy()
        exp_after = before.copy()
        for slot in (3, 5, 0, 15):
            exp_after[slot] = before[slot] + 1
        assert np.array_equal(after, exp_after), (step, after, exp_after)
    nvjsel.reset_rng_counters(table, [3, -1])
    assert int(table[3]) == 0 and int(table[5]) == 3


def test_repeated_calls_leave_workspace_clean():
    rng = np.random.default_rng(9)
    for trial in range(3):
        B, V = [4, 9, 2][trial], [3000, 777, 12000][trial]
        l = (rng.standard_normal((B, V)) * 2).astype(np.float32)
        T = [1.0] * B
        K = [int(x) for x in rng.choice([0, 5], B)]
        P = [float(x) for x in rng.choice([1.0, 0.8], B)]
        ids, used, keys = _sample(l, T, top_k=K, top_p=P)
        check_sampled(ids, used, T, K, P, keys, ctx=f"trial{trial}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_strided_rows_and_unaligned_vocab(dtype):
    """Rows taken from a wider buffer (row stride > V) and V not a multiple of
    the 16-byte vector: the scalar-load variants."""
    rng = np.random.default_rng(10)
    B, V, W = 5, 9001, 9016
    full = (rng.standard_normal((B, W)) * 2).astype(np.float32)
    lt = torch.from_numpy(full).to(dtype).cuda()[:, :V]
    assert lt.stride(0) == W
    keys = engine_keys(B, 3)
    T, K, P = [0.0, 0.8, 1.0, 0.5, 1.2], [0, 0, 30, 5, 0], [1.0, 1.0, 0.9, 1.0, 0.7]
    out = nvjsel.sample_token_ids(
        lt, torch.tensor(T, dtype=torch.float32).cuda(), keys_tensor(keys),
        top_k=torch.tensor(K, dtype=torch.int32).cuda(), top_p=torch.tensor(P, dtype=torch.float32).cuda())
    torch.cuda.synchronize()
    used = lt.float().cpu().numpy()
    check_sampled(out.cpu().numpy(), used, T, K, P, keys, ctx="strided")


def test_topk_clustered_in_one_chunk_takes_exact_path():
    """The row's top-k all sit in one 8192-element chunk: the row floor falls
    below that chunk's tier-A level, so the fast path must hand the row to the
    exact whole-row descent (and still agree with the oracle)."""
    rng = np.random.default_rng(21)
    B, V = 4, 248320
    l = rng.standard_normal((B, V)).astype(np.float32)
    for b in range(B):
        base = 8192 * (3 + b)
        l[b, base:base + 400] = 8.0 + rng.standard_normal(400).astype(np.float32)
    T = [1.0] * B
    K = [256, 100, 64, 256]
    P = [1.0, 0.9, 1.0, 0.8]
    ids, used, keys = _sample(l, T, top_k=K, top_p=P)
    check_sampled(ids, used, T, K, P, keys, ctx="clustered top-k")


def test_topp_crossing_bin_overflow_and_far_chunks():
    """Top-p-only rows whose crossing bin holds far more than the LDS list
    (200k equal values), rows with whole chunks far below the row maximum or
    all -inf (outside the 32-nat histogram window), in f32 and bf16."""
    rng = np.random.default_rng(22)
    B, V = 4, 248320
    l = np.full((B, V), -3.0, dtype=np.float32)
    l[0, rng.choice(V, 50, replace=False)] = 1.0          # crossing bin = the -3.0 plateau
    l[1] = rng.standard_normal(V).astype(np.float32)
    l[1, 8192 * 5:8192 * 9] = -200.0                        # chunks 40+ nats below the maximum
    l[2] = rng.standard_normal(V).astype(np.float32)
    l[2, 8192 * 2:8192 * 3] = -np.inf                      # a chunk of -inf
    l[3] = (rng.standard_normal(V) * 4).astype(np.float32)
    T = [1.0, 0.7, 1.0, 0.5]
    P = [0.5, 0.9, 0.95, 0.8]
    for dtype in (torch.float32, torch.bfloat16):
        ids, used, keys = _sample(l, T, top_k=[0] * B, top_p=P, dtype=dtype)
        check_sampled(ids, used, T, [0] * B, P, keys, ctx=f"top-p edges {dtype}")


def test_counter_table_gathers_before_scatter_across_rounds():
    """A slot repeated far apart in a large batch (past every 256-row block
    round): each row reads the counter as it was before the call."""
    table = torch.arange(0, 64, dtype=torch.int32).cuda() * 3
    B = 600
    rng = np.random.default_rng(31)
    slots = rng.integers(0, 64, B).astype(np.int32)
    slots[[5, 300, 599]] = 17  # 17 in three different 256-row rounds
    slots[[10, 520]] = -4      # slot 0 through the clamp
    slots[[7, 400]] = 90       # past the table: read its last entry, not written
    before = table.cpu().numpy().copy()
    keys = nvjsel.derive_rng_keys_from_table(torch.from_numpy(slots).cuda(), table)
    torch.cuda.synchronize()
    got = keys.cpu().numpy().view(np.uint32)
    for b, slot in enumerate(slots):
        s_eff = max(0, int(slot))
        exp = jr.engine_key(s_eff, int(before[min(s_eff, 63)]))
        assert tuple(int(x) for x in got[b]) == (int(exp[0]), int(exp[1])), b
    exp_after = before.copy()
    for slot in set(max(0, int(s)) for s in slots):
        if slot < 64:
            exp_after[slot] = before[slot] + 1
    assert np.array_equal(table.cpu().numpy(), exp_after)


def _bench_inputs(name):
    import bench

    return bench.make_inputs(torch, name, torch.device("cuda:0"))


@pytest.mark.parametrize("name", ["c2", "c3", "c5"])
def test_bench_workload_at_full_batch(name):
    """The exact inputs bench.py times (its seeded builders, same per-row
    parameter draws): C2 [8, 248320] f32, C3 [64, 248320] f32 (k=50, p=0.9,
    T=0.8) and C5 [256, 248320] bf16 with mixed per-row T / k / p -- every
    row checked against the oracle."""
    d = _bench_inputs(name)
    B = d["batch"]
    print(f"case {name} B={B}", flush=True)
    out = nvjsel.sample_token_ids(d["logits"], d["temperature"], d["keys"], top_k=d["top_k"], top_p=d["top_p"])
    torch.cuda.synchronize()
    used = d["logits"].float().cpu().numpy()
    keys = d["keys"].cpu().numpy().view(np.uint32)
    T = d["temperature"].cpu().numpy()
    K = d["top_k"].cpu().numpy() if d["top_k"] is not None else np.zeros(B, np.int32)
    P = d["top_p"].cpu().numpy() if d["top_p"] is not None else np.ones(B, np.float32)
    namb = check_sampled(out.cpu().numpy(), used, T, K, P, keys, ctx=name)
    assert namb <= max(1, B // 16)
    # the same call again on the reused workspace gives the same ids
    out2 = nvjsel.sample_token_ids(d["logits"], d["temperature"], d["keys"], top_k=d["top_k"], top_p=d["top_p"])
    assert torch.equal(out, out2)
