"""GPU parity of nvjsel_topk (jax.lax.top_k of the verifier route,
nanovllm_jax/model.py:893-898) against the oracle's ordering: values bitwise
equal to the input elements, indices by value descending then index
ascending.  Covers the candidate fast path, ties at the k-th value, rows that
need the exact full-row path (NaN, crowded ties), bf16/f16/f32 and strided
rows, and the lm_head_token_ids_and_topk caller with width > 1."""
import numpy as np
import pytest
import torch

import nvjsel
from oracle import selection as sel
from tests.gpu_helpers import check_greedy

pytestmark = pytest.mark.gpu

TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _check(logits: torch.Tensor, k: int, ctx: str):
    v, i = nvjsel.topk_hip(logits, k)
    torch.cuda.synchronize()
    x = logits.float().cpu().numpy()
    ev, ei = sel.topk(x, k)
    gi = i.cpu().numpy()
    assert np.array_equal(gi, ei), f"{ctx}: indices differ in rows {np.nonzero((gi != ei).any(1))[0][:5]}"
    assert np.array_equal(v.cpu().numpy().view(np.uint32), ev.view(np.uint32)), f"{ctx}: values differ"


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("batch,vocab,k", [(4, 4099, 1), (3, 4099, 7), (8, 248320, 2), (3, 248320, 50),
                                           (2, 248320, 256), (5, 300, 256)])
def test_topk_random(dt, batch, vocab, k):
    g = torch.Generator().manual_seed(batch * 1000 + k)
    x = (torch.randn(batch, vocab, generator=g) * 3).to(TORCH[dt]).cuda()
    _check(x, k, f"{dt} B={batch} V={vocab} k={k}")


def test_topk_zipf_rows_real_fixture():
    d = np.load("tests/golden/qwen08_logits_row.npz")
    row = torch.from_numpy(np.asarray(d["logits_0"], np.float32)).reshape(1, -1)
    _check(row.cuda(), 20, "qwen row")
    _check(row.to(torch.bfloat16).cuda(), 64, "qwen row bf16")


def test_topk_ties_at_threshold():
    g = torch.Generator().manual_seed(1)
    x = torch.randint(-50, 8, (6, 248320), generator=g).float()  # heavy ties everywhere
    _check(x.cuda(), 10, "int ties")
    _check(x.to(torch.bfloat16).cuda(), 256, "int ties bf16")


def test_topk_exact_row_path():
    """NaN rows and rows whose ties overflow the candidate lists."""
    x = torch.randn(4, 100000).float()
    x[0, 777] = float("nan")
    x[0, 5] = float("nan")
    x[1, :] = 1.5                       # every element tied
    x[2, 1000:] = -0.0                  # signed zeros tie with +0
    x[2, :1000] = 0.0
    x[3, 99999] = float("inf")
    _check(x.cuda(), 9, "exact path")


def test_topk_strided_rows():
    g = torch.Generator().manual_seed(2)
    big = torch.randn(5, 5000, generator=g).cuda()
    _check(big[:, :4099], 13, "strided")


def test_topk_rejects_bad_k():
    x = torch.zeros(2, 10).cuda()
    with pytest.raises(ValueError):
        nvjsel.topk_hip(x, 0)
    with pytest.raises(ValueError):
        nvjsel.topk_hip(x, 11)
    with pytest.raises(nvjsel.NvjselError):
        nvjsel.topk_hip(torch.zeros(2, 1000).cuda(), 257)


@pytest.mark.parametrize("top_k", [0, 5])
def test_lm_head_token_ids_and_topk_width(top_k):
    """model.py:833-898 with hidden [B, W, H], W = 3 (flattened to B*W rows)."""
    rng = np.random.default_rng(4)
    B, Wd, H, V = 2, 3, 1024, 4099
    h = sel.round_bf16(rng.normal(0, 1, (B, Wd, H)).astype(np.float32))
    E = sel.round_bf16(rng.normal(0, 0.02, (V, H)).astype(np.float32))
    ht = torch.from_numpy(h).to(torch.bfloat16).cuda()
    Et = torch.from_numpy(E).to(torch.bfloat16).cuda()
    ids, vals, idx = nvjsel.lm_head_token_ids_and_topk(ht, Et, top_k=top_k, weight_layout="vh")
    torch.cuda.synchronize()
    assert tuple(ids.shape) == (B, Wd)
    if top_k == 0:
        assert vals is None and idx is None
        check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(h.reshape(-1, H), E), 1, "width")
        return
    assert tuple(vals.shape) == (B, Wd, top_k) and tuple(idx.shape) == (B, Wd, top_k)
    # the route's dense logits come from the library (checked against float64
    # in test_lm_head_paths_gpu.py); top-k over them is bitwise
    logits = nvjsel.lm_head_logits_hip(ht.reshape(-1, H), Et, weight_layout="vh").float().cpu().numpy()
    ev, ei = sel.topk(logits, top_k)
    assert np.array_equal(idx.cpu().numpy().reshape(-1, top_k), ei)
    assert np.array_equal(vals.cpu().numpy().reshape(-1, top_k), ev)
    assert np.array_equal(ids.cpu().numpy().reshape(-1), ei[:, 0])


def test_topk_bench_workload_x2():
    """bench.py's x2 inputs (k=50 over [64, 248320] f32 Zipf rows), bitwise."""
    import bench

    d = bench.make_inputs(torch, "x2", torch.device("cuda:0"))
    vals, idx = nvjsel.topk_hip(d["logits"], d["k"])
    torch.cuda.synchronize()
    ev, ei = sel.topk(d["logits"].cpu().numpy(), d["k"])
    assert np.array_equal(idx.cpu().numpy(), ei)
    assert np.array_equal(vals.cpu().numpy().view(np.uint32), ev.view(np.uint32))
