"""GPU parity: fused LM-head greedy top-1 (libnvjsel) against the CPU oracle.

Mirrors the reference's checks (tests/test_lm_head_helpers.py:159-206: bf16
hidden [3,1,32] x E[257,32], V not a multiple of the tile) and extends them to
the BASELINE shapes (V=248320, H=1024) and every dispatch path."""
import numpy as np
import pytest
import torch

import nvjsel
from oracle import selection as sel
from tests.gpu_helpers import as_f32, bf16_tensor, check_greedy

pytestmark = pytest.mark.gpu


def _run(h, w, **kw):
    ids = nvjsel.lm_head_greedy_top1_hip(h, w, **kw)
    torch.cuda.synchronize()
    assert ids.dtype == torch.int32
    return ids.cpu().numpy().reshape(-1)


def test_reference_shape_tied_embedding_bf16():
    rng = np.random.default_rng(19)
    h = bf16_tensor(rng.standard_normal((3, 1, 32)))
    E = bf16_tensor(rng.standard_normal((257, 32)))
    ids = _run(h, E.T)  # the reference passes embed_tokens.T; used in place
    z = sel.lm_head_logits(as_f32(h)[:, 0], as_f32(E), weight_layout="vh")
    check_greedy(ids, z, 1, "ref-shape")
    assert ids.shape == (3,)


@pytest.mark.parametrize("batch", [1, 2, 5, 16, 17, 33, 64, 70])
def test_bf16_batches_odd_vocab(batch):
    rng = np.random.default_rng(100 + batch)
    H, V = 1024, 4099
    h = bf16_tensor(rng.standard_normal((batch, H)))
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.02)
    ids = _run(h, W, weight_layout="vh")
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    check_greedy(ids, z, 1, f"B={batch}")


def test_full_vocab_batch1_with_best_value():
    """hidden [1,1024] ~N(0,1), W [248320,1024] ~N(0,0.02), bf16."""
    g = torch.Generator().manual_seed(0)
    H, V = 1024, 248320
    h = torch.randn(1, H, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16)
    ids, best = nvjsel.lm_head_greedy_top1_hip(h.cuda(), W.cuda(), weight_layout="vh", return_best=True)
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.float().numpy(), W.float().numpy())
    check_greedy(ids.cpu().numpy(), z, 1, "C1")
    i = int(ids[0, 0])
    assert abs(float(best[0]) - sel.round_bf16(np.float32(z[0, i]))) <= 2 ** -7 * abs(z[0, i])


@pytest.mark.parametrize("batch", [1, 2, 20])
def test_f32_hidden_exact_split(batch):
    """f32 activations x bf16 weight: fp32 dot (no logit rounding), as jnp.dot promotes."""
    rng = np.random.default_rng(7 + batch)
    H, V = 512, 3001
    h = torch.from_numpy(rng.standard_normal((batch, H)).astype(np.float32)).cuda()
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    ids, best = nvjsel.lm_head_greedy_top1_hip(h, W, weight_layout="vh", return_best=True)
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.cpu().numpy(), as_f32(W))
    check_greedy(ids.cpu().numpy(), z, 0, "f32-hidden")
    zb = z[np.arange(batch), ids.cpu().numpy().reshape(-1)]
    assert np.allclose(best.cpu().numpy(), zb, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("layout", ["hv", "vh"])
@pytest.mark.parametrize("dt", [torch.float32, torch.float16])
def test_generic_paths(layout, dt):
    rng = np.random.default_rng(3)
    B, H, V = 4, 96, 777
    h = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).to(dt).cuda()
    Wvh = torch.from_numpy((rng.standard_normal((V, H)) * 0.1).astype(np.float32)).to(dt).cuda()
    W = Wvh if layout == "vh" else Wvh.T.contiguous()
    ids = _run(h, W, weight_layout=layout)
    z = sel.lm_head_logits(h.float().cpu().numpy(), Wvh.float().cpu().numpy())
    check_greedy(ids, z, 2 if dt == torch.float16 else 0, f"{layout}/{dt}")


def test_hidden_dim_not_multiple_of_32_uses_generic():
    rng = np.random.default_rng(5)
    h = bf16_tensor(rng.standard_normal((2, 1, 40)))
    E = bf16_tensor(rng.standard_normal((300, 40)))
    ids = _run(h, E.T)
    check_greedy(ids, sel.lm_head_logits(as_f32(h)[:, 0], as_f32(E)), 1, "H=40")


@pytest.mark.parametrize("H,B", [(256, 2), (512, 2), (512, 1), (1024, 5), (1024, 100), (256, 256)])
def test_ties_resolve_to_lowest_index_across_blocks(H, B):
    """Identical rows far apart in the vocabulary (different blocks/waves;
    B > 64: different blocked-GEMM tiles and lanes)."""
    rng = np.random.default_rng(11)
    V = 70000
    Wn = (rng.standard_normal((V, H)) * 0.01).astype(np.float32)
    h = np.abs(rng.standard_normal((B, H))).astype(np.float32)
    hot = np.full(H, 0.5, np.float32)
    for v in (65000, 40000, 12345, 69999):
        Wn[v] = hot
    ids = _run(bf16_tensor(h), bf16_tensor(Wn), weight_layout="vh")
    assert list(ids) == [12345] * B


@pytest.mark.parametrize("H,B", [(128, 3), (512, 3), (2048, 3), (512, 80), (1024, 130)])
def test_nan_logit_wins_first(H, B):
    rng = np.random.default_rng(12)
    V = 5000
    Wn = (rng.standard_normal((V, H)) * 0.01).astype(np.float32)
    Wn[4000, 3] = np.nan
    Wn[2500, 7] = np.nan
    ids = _run(bf16_tensor(rng.standard_normal((B, H))), bf16_tensor(Wn), weight_layout="vh")
    assert list(ids) == [2500] * B


def test_repeated_calls_reuse_workspace():
    rng = np.random.default_rng(13)
    H, V = 256, 9000
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    for trial in range(4):
        B = [3, 40, 1, 16][trial]
        h = bf16_tensor(rng.standard_normal((B, H)))
        ids = _run(h, W, weight_layout="vh")
        check_greedy(ids, sel.lm_head_logits(as_f32(h), as_f32(W)), 1, f"trial{trial}")


@pytest.mark.parametrize("H", [512, 1024, 2048])
@pytest.mark.parametrize("batch", [1, 2])
def test_streaming_gemv_shapes(H, batch):
    """The small-batch streaming kernel (H a multiple of 512), odd vocab tail."""
    rng = np.random.default_rng(H + batch)
    V = 10007
    h = bf16_tensor(rng.standard_normal((batch, H)))
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.03)
    ids, best = nvjsel.lm_head_greedy_top1_hip(h, W, weight_layout="vh", return_best=True)
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    check_greedy(ids.cpu().numpy(), z, 1, f"gemv H={H} B={batch}")


@pytest.mark.parametrize("batch", [1, 2, 5, 16, 20, 32, 33, 64, 70])
def test_fused_lm_head_sample(batch):
    """nvjsel_lm_head_sample vs the oracle: greedy rows, temperature rows (JAX keys)."""
    from tests.gpu_helpers import check_fused_sampled, engine_keys, keys_tensor

    rng = np.random.default_rng(500 + batch)
    H, V = 1024, 20011
    h = bf16_tensor(rng.standard_normal((batch, H)))
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    T = [float(x) for x in rng.choice([0.0, 0.7, 1.0, 1.5], batch)]
    keys = engine_keys(batch, 11)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    namb = check_fused_sampled(ids.cpu().numpy(), z, T, keys, 1, f"fused B={batch}")
    assert namb <= max(1, batch // 8)


def test_fused_lm_head_sample_full_vocab_c4():
    """hidden [64,1024] bf16 ~N(0,1), W [248320,1024] ~N(0,0.02), T=1."""
    from tests.gpu_helpers import check_fused_sampled, engine_keys, keys_tensor

    g = torch.Generator().manual_seed(3)
    B, H, V = 64, 1024, 248320
    h = torch.randn(B, H, generator=g).to(torch.bfloat16)
    W = (torch.randn(V, H, generator=g) * 0.02).to(torch.bfloat16)
    keys = engine_keys(B, 5)
    ids = nvjsel.lm_head_sample_token_ids(h.cuda(), W.cuda(), temperatures=torch.ones(B).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    z = sel.lm_head_logits(h.float().numpy(), W.float().numpy())
    namb = check_fused_sampled(ids.cpu().numpy(), z, [1.0] * B, keys, 1, "C4")
    assert namb <= 4


@pytest.mark.parametrize("batch", [20, 64])
def test_fused_lm_head_sample_nan_rows_fill_queue(batch):
    """Rows whose hidden holds a NaN have NaN logits everywhere: every entry
    scores +inf approximately, so each one stays a candidate, the epilogue's
    candidate queue overflows and is rescored exactly mid-run (several times
    at V=20011); those rows take the first index (first NaN wins, as
    jnp.argmax), and the finite rows beside them stay exact."""
    from tests.gpu_helpers import check_fused_sampled, engine_keys, keys_tensor

    rng = np.random.default_rng(900 + batch)
    H, V = 1024, 20011
    hn = rng.standard_normal((batch, H))
    nan_rows = [1, batch // 2, batch - 1]
    for b in nan_rows:
        hn[b, 17] = np.nan
    h = bf16_tensor(hn)
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.05)
    T = [1.0] * batch
    keys = engine_keys(batch, 23)
    ids = nvjsel.lm_head_sample_token_ids(h, W, temperatures=torch.tensor(T).cuda(),
                                          rng_keys=keys_tensor(keys), weight_layout="vh")
    torch.cuda.synchronize()
    got = ids.cpu().numpy()
    assert [int(got[b]) for b in nan_rows] == [0] * len(nan_rows)
    z = sel.lm_head_logits(as_f32(h), as_f32(W))
    namb = check_fused_sampled(got, z, T, keys, 1, f"fused NaN rows B={batch}")
    assert namb <= max(1, batch // 8)


@pytest.mark.parametrize("seq_len", [1, 3])
def test_mtp_draft_top1_casts_and_flattens(seq_len):
    """mtp/mtp_layer.py:220-248: fp32 x_normed [B, T, H] cast to the weight's
    bf16, T > 1 flattened to B*T rows and reshaped to [B, T]."""
    rng = np.random.default_rng(40 + seq_len)
    B, H, V = 2, 1024, 4099
    x = rng.standard_normal((B, seq_len, H)).astype(np.float32)
    W = bf16_tensor(rng.standard_normal((V, H)) * 0.02)
    ids = nvjsel.mtp_greedy_top1_token_ids(torch.from_numpy(x).cuda(), W, weight_layout="vh")
    torch.cuda.synchronize()
    assert tuple(ids.shape) == (B, seq_len) and ids.dtype == torch.int32
    xb = sel.round_bf16(x.reshape(-1, H))  # the cast the contract requires
    check_greedy(ids.cpu().numpy().reshape(-1), sel.lm_head_logits(xb, as_f32(W)), 1, f"mtp T={seq_len}")


@pytest.mark.parametrize("name", ["c1", "c4", "x7"])
def test_last_block_reduce_is_consistent_over_1000_calls(name):
    """The cross-block reduce (per-row atomicMax, then the last block by ticket
    writes the ids and re-zeroes the workspace) at the C1 / C4 shapes and the
    B = 256 fused Gumbel shape of the blocked GEMM (x7): 1,000
    back-to-back launches on one workspace must all return the first call's
    ids.  Each launch writes its own output row; the first mismatch is named."""
    import bench
    from nvjsel import _lib

    dev = torch.device("cuda:0")
    d = bench.make_inputs(torch, name, dev)
    W = bench.lm_weight(torch, dev)
    B, N = d["batch"], 1000
    lib = _lib.load()
    out = torch.full((N, B), -1, dtype=torch.int32, device=dev)
    ws = torch.zeros(lib.nvjsel_lm_head_workspace_size(B), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    h = d["hidden"]
    for i in range(N):
        o = out[i].data_ptr()
        if name == "c1":
            _lib.call("nvjsel_lm_head_top1", h.data_ptr(), 1, W.data_ptr(), 1, 0, B, 1024, W.shape[0], 1, o, None,
                      ws.data_ptr(), ws.numel(), stream)
        else:
            _lib.call("nvjsel_lm_head_sample", h.data_ptr(), 1, W.data_ptr(), 1, 0, B, 1024, W.shape[0], 1,
                      d["temperature"].data_ptr(), d["keys"].data_ptr(), o, ws.data_ptr(), ws.numel(), stream)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    bad = np.nonzero((got != got[0]).any(axis=1))[0]
    assert bad.size == 0, f"call {bad[0]} differs from call 0: {got[bad[0]][:8]} vs {got[0][:8]}"
    assert np.all((got[0] >= 0) & (got[0] < W.shape[0]))
    assert not ws.any().item()  # the workspace is zero at rest
