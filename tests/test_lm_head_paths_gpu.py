"""GPU parity of the LM-head paths added for the reference's other operating
points, against the float64 oracle:

* the [H, V] weight layout (the reference's materialised lm_head,
  configs/server/gpu_optimal.yaml:56, load_weights.py:256-258; the layout
  lm_head_triton.py:51-55 reads) -- the streaming [H, V] kernel, B <= 8 per
  launch;
* fp32 activations (lm_head_decode_act_dtype's default, config.py:120;
  model.py:277-285) at 3 <= B <= 8 on the [V, H] table -- one W pass, exact
  fp32 products;
* dense logits (nvjsel_lm_head_logits) on every path, and the routes built on
  them: top-k values / indices (model.py:866-898) and top-k / top-p sampling
  from the hidden state -- no vendor GEMM.
"""
import numpy as np
import pytest
import torch

import nvjsel
from oracle import selection as sel
from tests.gpu_helpers import (as_f32, bf16_tensor, check_fused_sampled, check_greedy, check_sampled,
                               engine_keys, keys_tensor)

pytestmark = pytest.mark.gpu


def _hidden(rng, B, H, dtype):
    h = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda()
    return h.to(dtype)


def _check_logits(got: torch.Tensor, h: np.ndarray, w_vh: np.ndarray, rc: int, ctx: str):
    """Logits against the float64 dot z = h . w.  An fp32 accumulation of H
    products (any order) is within H * 2^-24 * A of z, A = sum |h_k w_k|
    (the standard summation bound); the rounding (rc) adds at most half an
    ulp of the rounded value.  Almost every value must also equal the
    rounded exact logit."""
    h64, w64 = np.asarray(h, np.float64), np.asarray(w_vh, np.float64)
    z64 = h64 @ w64.T
    A = np.abs(h64) @ np.abs(w64).T
    H = h64.shape[1]
    g = got.float().cpu().numpy().astype(np.float64)
    assert g.shape == z64.shape, ctx
    acc = H * 2.0 ** -24 * A
    if rc == 0:
        err = np.abs(g - z64)
        assert np.all(err <= acc + 1e-30), (ctx, float((err / (acc + 1e-30)).max()))
        return
    rnd = sel.round_bf16 if rc == 1 else sel.round_f16
    half_ulp = (2.0 ** -8 if rc == 1 else 2.0 ** -11) * np.abs(g)
    err = np.abs(g - z64)
    assert np.all(err <= acc + half_ulp + 1e-30), (ctx, float((err / (acc + half_ulp + 1e-30)).max()))
    exp = rnd(z64.astype(np.float32)).astype(np.float64)
    frac = float(np.mean(g == exp))
    assert frac > 0.995, (ctx, frac)


@pytest.mark.parametrize("B", [1, 2, 3, 5, 8, 13])
@pytest.mark.parametrize("act", [torch.bfloat16, torch.float32])
def test_hv_layout_greedy(B, act):
    rng = np.random.default_rng(100 + B)
    H, V = 1024, 20008
    Wvh = (rng.standard_normal((V, H)) * 0.03).astype(np.float32)
    Whv = torch.from_numpy(Wvh.T.copy()).cuda().to(torch.bfloat16)  # [H, V] contiguous
    h = _hidden(rng, B, H, act)
    ids = nvjsel.lm_head_greedy_top1_hip(h, Whv, weight_layout="hv")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.float().cpu().numpy(), Whv.float().cpu().numpy(), weight_layout="hv")
    rc = 1 if act == torch.bfloat16 else 0
    check_greedy(ids.cpu().numpy().reshape(-1), z, rc, f"hv B={B} {act}")


@pytest.mark.parametrize("H", [256, 512, 100])
def test_hv_layout_other_hidden_sizes(H):
    rng = np.random.default_rng(H)
    B, V = 4, 3000
    Whv = bf16_tensor(rng.standard_normal((H, V)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    ids = nvjsel.lm_head_greedy_top1_hip(h, Whv, weight_layout="hv")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(Whv), weight_layout="hv")
    check_greedy(ids.cpu().numpy().reshape(-1), z, 1, f"hv H={H}")


def test_hv_layout_sample():
    rng = np.random.default_rng(7)
    B, H, V = 6, 1024, 20008
    Whv = bf16_tensor(rng.standard_normal((H, V)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    T = [0.0, 0.7, 1.0, 1.5, 0.0, 1.0]
    keys = engine_keys(B, 9)
    ids = nvjsel.lm_head_sample_token_ids(h, Whv, temperatures=torch.tensor(T).cuda(), rng_keys=keys_tensor(keys),
                                          weight_layout="hv")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(Whv), weight_layout="hv")
    assert check_fused_sampled(ids.cpu().numpy(), z, T, keys, 1, "hv sample") <= 1


@pytest.mark.parametrize("B", [1, 8])
def test_hv_layout_full_vocab(B):
    """The promoted serving layout at the BASELINE shape: W [1024, 248320] bf16."""
    import bench

    dev = torch.device("cuda:0")
    Whv = bench.lm_weight(torch, dev).T.contiguous()
    g = torch.Generator(device=dev)
    g.manual_seed(50 + B)
    h = torch.randn(B, 1024, device=dev, generator=g).to(torch.bfloat16)
    ids = nvjsel.lm_head_greedy_top1_hip(h, Whv, weight_layout="hv")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(Whv), weight_layout="hv")
    check_greedy(ids.cpu().numpy().reshape(-1), z, 1, f"hv full B={B}")


@pytest.mark.parametrize("B", [3, 4, 6, 8])
def test_fp32_activations_one_pass(B):
    """fp32 hidden x bf16 [V, H] (the reference's default decode activation):
    fp32 logits, no rounding."""
    rng = np.random.default_rng(200 + B)
    H, V = 1024, 30011
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.03)
    h = _hidden(rng, B, H, torch.float32)
    ids = nvjsel.lm_head_greedy_top1_hip(h, W, weight_layout="vh")
    torch.cuda.synchronize()
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(as_f32(h), as_f32(W)), 0, f"f32 act B={B}")


def test_fp32_activations_full_vocab_b8():
    import bench

    dev = torch.device("cuda:0")
    W = bench.lm_weight(torch, dev)
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    h = torch.randn(8, 1024, device=dev, generator=g)
    ids = nvjsel.lm_head_greedy_top1_hip(h, W, weight_layout="vh")
    torch.cuda.synchronize()
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(as_f32(h), as_f32(W)), 0, "f32 act full B=8")


def test_fp32_activations_sample():
    rng = np.random.default_rng(3)
    B, H, V = 7, 1024, 20011
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.float32)
    T = [1.0, 0.0, 0.6, 1.0, 2.0, 0.8, 1.0]
    keys = engine_keys(B, 4)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(), rng_keys=keys_tensor(keys),
                                          weight_layout="vh")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    assert check_fused_sampled(ids.cpu().numpy(), z, T, keys, 0, "f32 act sample") <= 1


# (B, H, layout, act, weight dtype): streaming [V,H] B<=2, fp32 B<=8, tile 3..64 and
# 64-row chunks, [H,V], f16 MFMA, generic (H not a multiple of 32)
LOGIT_CASES = [
    (1, 1024, "vh", torch.bfloat16, torch.bfloat16),
    (2, 512, "vh", torch.float32, torch.bfloat16),
    (6, 1024, "vh", torch.float32, torch.bfloat16),
    (40, 1024, "vh", torch.bfloat16, torch.bfloat16),
    (70, 1024, "vh", torch.bfloat16, torch.bfloat16),
    (5, 1024, "hv", torch.bfloat16, torch.bfloat16),
    (11, 1024, "hv", torch.float32, torch.bfloat16),
    (20, 1024, "vh", torch.float32, torch.bfloat16),
    (9, 256, "vh", torch.float16, torch.float16),
    (3, 40, "vh", torch.bfloat16, torch.bfloat16),
]


@pytest.mark.parametrize("B,H,layout,act,wdt", LOGIT_CASES)
def test_dense_logits_match_float64(B, H, layout, act, wdt):
    rng = np.random.default_rng(B * 1000 + H)
    V = 5008
    Wvh = torch.from_numpy((rng.standard_normal((V, H)) * 0.05).astype(np.float32)).to(wdt).cuda()
    W = Wvh if layout == "vh" else Wvh.T.contiguous()
    h = _hidden(rng, B, H, act)
    logits = nvjsel.lm_head_logits_hip(h, W, weight_layout=layout)
    torch.cuda.synchronize()
    rc = nvjsel.reference_reduce_cast(act, wdt)
    # the dtype jnp.dot returns: bf16 x bf16 -> bf16, f16 x f16 -> f16, else f32
    assert logits.dtype == {1: torch.bfloat16, 2: torch.float16}.get(rc, torch.float32)
    _check_logits(logits, h.float().cpu().numpy(), Wvh.float().cpu().numpy(), rc, f"{B},{H},{layout},{act},{wdt}")


@pytest.mark.parametrize("top_k", [1, 8, 50])
@pytest.mark.parametrize("layout", ["vh", "hv"])
def test_lm_head_topk_route_native(top_k, layout):
    """lm_head_token_ids_and_topk(top_k > 0): the library's logits (checked
    against float64) and lax.top_k order over them, bitwise."""
    rng = np.random.default_rng(top_k)
    B, H, V = 6, 1024, 30008
    Wvh = bf16_tensor(rng.standard_normal((V, H)) * 0.03)
    W = Wvh if layout == "vh" else Wvh.T.contiguous()
    h = _hidden(rng, B, H, torch.bfloat16)
    ids, vals, idx = nvjsel.lm_head_token_ids_and_topk(h[:, None, :], W, top_k=top_k, weight_layout=layout)
    logits = nvjsel.lm_head_logits_hip(h, W, weight_layout=layout)
    torch.cuda.synchronize()
    _check_logits(logits, as_f32(h), as_f32(Wvh), 1, "topk route logits")
    ev, ei = sel.topk(logits.float().cpu().numpy(), top_k)
    assert np.array_equal(idx.cpu().numpy().reshape(B, top_k), ei)
    assert np.array_equal(vals.cpu().numpy().reshape(B, top_k).view(np.uint32), ev.view(np.uint32))
    assert np.array_equal(ids.cpu().numpy().reshape(-1), ei[:, 0])


def test_hidden_to_filtered_sampling_native():
    """lm_head_sample_token_ids with top_k / top_p: library logits, then the
    sampler; ids against the oracle over the same logits."""
    rng = np.random.default_rng(11)
    B, H, V = 8, 1024, 30008
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    T = [0.0, 0.7, 1.0, 1.0, 0.9, 1.2, 0.5, 1.0]
    K = [0, 20, 0, 100, 5, 0, 50, 0]
    P = [1.0, 1.0, 0.9, 0.8, 1.0, 0.95, 0.7, 1.0]
    keys = engine_keys(B, 2)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(), rng_keys=keys_tensor(keys),
                                          top_k=torch.tensor(K, dtype=torch.int32).cuda(),
                                          top_p=torch.tensor(P).cuda(), weight_layout="vh")
    logits = nvjsel.lm_head_logits_hip(h, W, weight_layout="vh")
    torch.cuda.synchronize()
    _check_logits(logits, as_f32(h), as_f32(W), 1, "filtered sampling logits")
    check_sampled(ids.cpu().numpy(), logits.float().cpu().numpy(), T, K, P, keys, ctx="hidden->filtered")


# Blocked GEMM (bf16 activations, [V, H] bf16): one pass over W per 256 rows,
# greedy and logits, above 64 rows -- above 128 where the tile kernel serves
# the shape (H = 1024; B = 65 and 128 take 64-row tile passes); B = 300 takes
# a 256-row and a 44-row launch; B = 160 the kernel that skips padding waves.
@pytest.mark.parametrize("B,H", [(65, 1024), (128, 1024), (160, 1024), (256, 1024), (300, 512), (100, 2048),
                                 (77, 64)])
def test_gemm_greedy_and_logits(B, H):
    rng = np.random.default_rng(7000 + B + H)
    V = 10000 + (B % 7)  # not a multiple of the 128-row tile
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    ids = nvjsel.lm_head_greedy_top1_hip(h, W.T)
    logits = nvjsel.lm_head_logits_hip(h, W.T)
    torch.cuda.synchronize()
    hf, wf = h.float().cpu().numpy(), W.float().cpu().numpy()
    z = sel.lm_head_logits(hf, wf)
    check_greedy(ids.cpu().numpy().reshape(-1), z, 1, f"gemm B={B} H={H}")
    _check_logits(logits, hf, wf, 1, f"gemm logits B={B} H={H}")
    # a second call on the same workspace (its keys are cleared at rest)
    ids2 = nvjsel.lm_head_greedy_top1_hip(h, W.T)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2)


@pytest.mark.parametrize("B,H", [(33, 1024), (64, 1024), (65, 512), (81, 1024), (100, 1024), (200, 1024),
                                 (300, 1024), (32, 1024)])
def test_gemm_f32_activations(B, H):
    """fp32 activations (lm_head_decode_act_dtype fp32) above 32 rows: the
    blocked GEMM on three bf16 terms per value (the narrow layout up to 64
    rows; at H = 1024 and 65-128 rows 64-row narrow passes, then 16-row tile
    passes and the GEMV for a last row: B = 81, 100) -- one pass over W per
    256 rows, greedy and logits -- against the float64 dot (fp32 logits); 32
    rows take two 16-row tile passes."""
    rng = np.random.default_rng(7700 + B + H)
    V = 9001
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.float32)
    ids = nvjsel.lm_head_greedy_top1_hip(h, W.T)
    logits = nvjsel.lm_head_logits_hip(h, W.T)
    torch.cuda.synchronize()
    assert logits.dtype == torch.float32
    hf, wf = h.cpu().numpy(), W.float().cpu().numpy()
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(hf, wf), 0, f"gemm f32 B={B} H={H}")
    _check_logits(logits, hf, wf, 0, f"gemm f32 logits B={B} H={H}")


@pytest.mark.parametrize("B", [33, 60, 85, 300])
def test_gemm_sample_f32_activations(B):
    """Fused Gumbel sampling with fp32 activations at 33-64 rows (the narrow
    layout, 32-wide K stages) and above 80 rows (the full layout, 16-wide K
    stages; B = 300: two 256-row passes) -- the blocked GEMM on three bf16
    terms -- greedy rows beside temperature rows, against the oracle's scores
    on the float64 logits (fp32 logits, no rounding)."""
    rng = np.random.default_rng(9300 + B)
    H, V = 1024, 12007
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.float32)
    T = [float(x) for x in rng.choice([0.0, 0.6, 1.0], B)]
    keys = engine_keys(B, 77 + B)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.cpu().numpy(), W.float().cpu().numpy())
    namb = check_fused_sampled(ids.cpu().numpy(), z, T, keys, 0, f"gemm f32 sample B={B}")
    assert namb <= max(1, B // 16)


def test_gemm_f32_activations_with_prenorm():
    """The reference's default decode configuration at a serving batch: the
    final RMSNorm into fp32 activations (prologue kernel), then the GEMM on
    three bf16 terms, B = 256, V = 151936."""
    rng = np.random.default_rng(4343)
    B, H, V = 256, 1024, 151936
    x = sel.round_bf16(rng.normal(0.0, 3.0, (B, H)).astype(np.float32))
    nw = rng.normal(0.0, 0.2, H).astype(np.float32)
    W = sel.round_bf16(rng.normal(0.0, 0.02, (V, H)).astype(np.float32))
    ids = nvjsel.lm_head_greedy_top1_hip(
        torch.from_numpy(x).to(torch.bfloat16).cuda(), torch.from_numpy(W).to(torch.bfloat16).cuda(),
        weight_layout="vh", norm_weight=torch.from_numpy(nw).cuda(), rms_norm_eps=1e-6, act_dtype=torch.float32)
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype="bf16", act_dtype="f32")
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(xin, W), 0, "gemm f32 B=256 prenorm")


@pytest.mark.parametrize("B,H,act", [(9, 1024, torch.bfloat16), (17, 1024, torch.bfloat16), (64, 512, torch.bfloat16),
                                     (65, 1024, torch.bfloat16), (300, 1024, torch.bfloat16), (48, 1024, torch.float32),
                                     (25, 512, torch.float32)])
def test_gemm_hv_weights(B, H, act):
    """[H, V] weights (vocabulary contiguous: the reference's materialised
    lm_head operand) above the 8-row streaming kernel: the blocked GEMM with
    row-major W stages and transposing LDS reads, greedy and logits, a
    vocabulary whose last 256-column tile is partial (V % 256 = 16)."""
    rng = np.random.default_rng(7900 + B + H)
    V = 10000
    Whv = bf16_tensor(rng.standard_normal((H, V)) * 0.05)  # contiguous [H, V]
    h = _hidden(rng, B, H, act)
    ids = nvjsel.lm_head_greedy_top1_hip(h, Whv)
    logits = nvjsel.lm_head_logits_hip(h, Whv)
    torch.cuda.synchronize()
    rc = 1 if act == torch.bfloat16 else 0
    hf, wf = h.float().cpu().numpy(), Whv.float().cpu().numpy().T.copy()
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(hf, wf), rc, f"gemm hv B={B} H={H}")
    _check_logits(logits, hf, wf, rc, f"gemm hv logits B={B} H={H}")


def test_gemm_hv_greedy_winner_in_last_columns():
    """The greedy maximum in the last 8 columns of a partial last tile: the
    re-read groups past V duplicate those columns and must not win."""
    rng = np.random.default_rng(7999)
    B, H, V = 40, 512, 4104  # V % 256 = 8
    Whv = rng.standard_normal((H, V)) * 0.02
    h = rng.standard_normal((B, H)).astype(np.float32)
    for b in range(B):  # row b's winner at column V - 1 - (b % 8)
        Whv[:, V - 1 - (b % 8)] += 0.5 * h[b] / np.linalg.norm(h[b])
    Wt = bf16_tensor(Whv)
    ht = torch.from_numpy(h).cuda().to(torch.bfloat16)
    ids = nvjsel.lm_head_greedy_top1_hip(ht, Wt)
    torch.cuda.synchronize()
    z = sel.lm_head_logits(ht.float().cpu().numpy(), Wt.float().cpu().numpy().T.copy())
    check_greedy(ids.cpu().numpy().reshape(-1), z, 1, "gemm hv last columns")
    assert np.all(ids.cpu().numpy().reshape(-1) < V)


@pytest.mark.parametrize("B,act", [(130, torch.bfloat16), (100, torch.float32)])
def test_gemm_hv_matches_vh_bitwise(B, act):
    """Where both layouts run the blocked GEMM (bf16 above 64 rows; fp32
    activations at 100 rows: two narrow passes on either layout), the [H, V] kernel multiplies the same products
    in the same k order as the [V, H] one: logits bitwise equal, sampled ids
    equal."""
    rng = np.random.default_rng(9600 + B)
    H, V = 1024, 12008
    Wvh = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    Whv = Wvh.T.contiguous()
    h = _hidden(rng, B, H, act)
    T = torch.tensor([float(x) for x in rng.choice([0.0, 0.7, 1.0], B)]).cuda()
    keys = keys_tensor(engine_keys(B, 56 + B))
    la = nvjsel.lm_head_logits_hip(h, Whv)
    lb = nvjsel.lm_head_logits_hip(h, Wvh.T)
    assert torch.equal(la, lb)
    ga = nvjsel.lm_head_greedy_top1_hip(h, Whv)
    gb = nvjsel.lm_head_greedy_top1_hip(h, Wvh.T)
    assert torch.equal(ga, gb)
    ia = nvjsel.lm_head_sample_token_ids(h, Whv, temperatures=T, rng_keys=keys)
    ib = nvjsel.lm_head_sample_token_ids(h, Wvh, temperatures=T, rng_keys=keys, weight_layout="vh")
    torch.cuda.synchronize()
    assert torch.equal(ia, ib)


@pytest.mark.parametrize("B,act", [(12, torch.bfloat16), (20, torch.bfloat16), (130, torch.bfloat16),
                                   (12, torch.float32), (30, torch.float32), (64, torch.float32)])
def test_gemm_hv_sample(B, act):
    """Fused Gumbel sampling through the [H, V] blocked GEMM (above 8 rows;
    the narrow layout up to 64 rows), greedy
    rows beside temperature rows.
    Rows whose kernel id differs within the rounding-flip exemption are
    listed in the terminal summary."""
    rng = np.random.default_rng(9500 + B)
    H, V = 1024, 12008
    Whv = bf16_tensor(rng.standard_normal((H, V)) * 0.05)
    h = _hidden(rng, B, H, act)
    T = [float(x) for x in rng.choice([0.0, 0.7, 1.0], B)]
    keys = engine_keys(B, 55 + B)
    ids = nvjsel.lm_head_sample_token_ids(h, Whv, temperatures=torch.tensor(T).cuda(), rng_keys=keys_tensor(keys))
    torch.cuda.synchronize()
    rc = 1 if act == torch.bfloat16 else 0
    z = sel.lm_head_logits(h.float().cpu().numpy(), Whv.float().cpu().numpy().T.copy())
    namb = check_fused_sampled(ids.cpu().numpy(), z, T, keys, rc, f"gemm hv sample B={B}")
    from tests.gpu_helpers import REPORTS
    assert namb <= max(2, B // 16), REPORTS[-1:]


@pytest.mark.parametrize("rc", [0, 2])
def test_gemm_other_roundings(rc):
    """The blocked GEMM with the caller's reduce_cast: 0 (fp32 logits, f32
    out) and 2 (f16 rounding), greedy and logits."""
    rng = np.random.default_rng(880 + rc)
    B, H, V = 96, 512, 7001
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    ids = nvjsel.lm_head_greedy_top1_hip(h, W.T, reduce_cast=rc)
    logits = nvjsel.lm_head_logits_hip(h, W.T, reduce_cast=rc)
    torch.cuda.synchronize()
    hf, wf = h.float().cpu().numpy(), W.float().cpu().numpy()
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(hf, wf), rc, f"gemm rc={rc}")
    _check_logits(logits, hf, wf, rc, f"gemm logits rc={rc}")


def test_gemm_full_vocab_b256_with_prenorm():
    """The bench shape (B = 256, V = 151936, H = 1024) through the final-norm
    entry (prologue kernel into the workspace, then the GEMM), against the
    oracle's norm + float64 LM head."""
    rng = np.random.default_rng(4242)
    B, H, V = 256, 1024, 151936
    x = sel.round_bf16(rng.normal(0.0, 3.0, (B, H)).astype(np.float32))
    nw = rng.normal(0.0, 0.2, H).astype(np.float32)
    W = sel.round_bf16(rng.normal(0.0, 0.02, (V, H)).astype(np.float32))
    ids = nvjsel.lm_head_greedy_top1_hip(
        torch.from_numpy(x).to(torch.bfloat16).cuda(), torch.from_numpy(W).to(torch.bfloat16).cuda(),
        weight_layout="vh", norm_weight=torch.from_numpy(nw).cuda(), rms_norm_eps=1e-6, act_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype="bf16", act_dtype="bf16")
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(xin, W), 1, "gemm B=256 prenorm")


@pytest.mark.parametrize("B,H", [(65, 512), (130, 1024), (200, 1024), (256, 1024), (300, 1024), (513, 512)])
def test_gemm_sample_mixed_temperatures(B, H):
    """Fused Gumbel sampling through the blocked GEMM (above 64 rows, above
    192 where the tile kernel serves H = 1024: B = 130 takes 64-row tile
    passes; B = 300 and 513 take two and three 256-row passes that reuse the
    row keys and the ticket): greedy rows (T = 0) beside temperature rows, a
    vocabulary that is not a multiple of the 256-row tile, against the
    oracle's scores s_v = rnd(z_v)/T + g_v."""
    rng = np.random.default_rng(9100 + B + H)
    V = 20011
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    T = [float(x) for x in rng.choice([0.0, 0.5, 1.0, 1.7], B)]
    keys = engine_keys(B, 31 + B)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.float().cpu().numpy(), W.float().cpu().numpy())
    namb = check_fused_sampled(ids.cpu().numpy(), z, T, keys, 1, f"gemm sample B={B} H={H}")
    assert namb <= max(1, B // 16)
    # a second call on the same inputs draws the same ids
    ids2 = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                           rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2)


def test_gemm_sample_nan_rows_fill_queue():
    """NaN hidden rows score +inf everywhere, so every one of their entries
    stays a candidate: the per-wave candidate queue of the GEMM's sample
    epilogue fills, is compacted and rescored exactly mid-tile many times.
    Those rows take index 0 (first NaN wins); the finite rows stay exact."""
    rng = np.random.default_rng(9300)
    B, H, V = 200, 1024, 30011
    hn = rng.standard_normal((B, H))
    nan_rows = [0, 33, 64, 127, 199]
    for b in nan_rows:
        hn[b, 5] = np.nan
    h = bf16_tensor(hn)
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    T = [1.0] * B
    keys = engine_keys(B, 47)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    assert [int(got[b]) for b in nan_rows] == [0] * len(nan_rows)
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    namb = check_fused_sampled(got, z, T, keys, 1, "gemm sample NaN rows")
    assert namb <= max(1, B // 16)


def test_gemm_sample_bench_workload_b256():
    """The timed x7 workload (fused LM-head + Gumbel, B = 256, V = 248320,
    T = 1, engine keys), built as the bench builds it, against the oracle."""
    import bench

    dev = torch.device("cuda:0")
    W = bench.lm_weight(torch, dev)
    d = bench.make_inputs(torch, "x7", dev)
    B, h, t, kt = d["batch"], d["hidden"], d["temperature"], d["keys"]
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=t, rng_keys=kt, weight_layout="vh")
    torch.cuda.synchronize()
    keys = [tuple(int(x) & 0xFFFFFFFF for x in row) for row in kt.cpu().numpy().reshape(B, 2)]
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    namb = check_fused_sampled(ids.cpu().numpy(), z, t.cpu().numpy().tolist(), keys, 1, "x7 B=256")
    assert namb <= 8


@pytest.mark.parametrize("rc", [0, 2])
def test_gemm_sample_other_roundings(rc):
    """Sample mode of the blocked GEMM with fp32 (0) and f16 (2) rounding of
    the logits before the draws, greedy rows beside temperature rows."""
    rng = np.random.default_rng(9500 + rc)
    B, H, V = 100, 1024, 12007
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    h = _hidden(rng, B, H, torch.bfloat16)
    T = [float(x) for x in rng.choice([0.0, 0.8, 1.0], B)]
    keys = engine_keys(B, 71 + rc)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh", reduce_cast=rc)
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.float().cpu().numpy(), W.float().cpu().numpy())
    namb = check_fused_sampled(ids.cpu().numpy(), z, T, keys, rc, f"gemm sample rc={rc}")
    assert namb <= max(1, B // 16)
