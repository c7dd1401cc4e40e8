"""GPU parity of the final-RMSNorm prologue (hidden_is_normed=False,
nanovllm_jax/model.py:734-762 with rms_norm, layers.py:11-29) in front of the
LM head, on every dispatch path: streaming GEMV and bf16 tile kernel (fused in
the launch), MFMA split / generic paths (prologue kernel into the workspace).

The checker is the oracle's lm_head_input followed by float64 logits; rows
whose top-2 logits are within the accumulation/rounding margin are accepted on
the admissible set, as in the other LM-head tests."""
import numpy as np
import pytest
import torch

import nvjsel
from oracle import selection as sel
from tests.gpu_helpers import check_fused_sampled, check_greedy, engine_keys, keys_tensor

pytestmark = pytest.mark.gpu

TORCH = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
RC = {("bf16", "bf16"): 1, ("f16", "f16"): 2}


def _inputs(rng, batch, H, V, hidden_dtype):
    x = rng.normal(0.0, 3.0, (batch, H)).astype(np.float32)
    x = sel.lm_head_input(x, None, act_dtype=hidden_dtype)  # representable in hidden_dtype
    nw = rng.normal(0.0, 0.2, H).astype(np.float32)
    W = sel.round_bf16(rng.normal(0.0, 0.02, (V, H)).astype(np.float32))
    return x, nw, W


@pytest.mark.parametrize("batch,H,hidden_dtype,act_dtype", [
    (1, 1024, "bf16", "bf16"),   # streaming GEMV, fused
    (2, 1024, "f32", "f32"),     # streaming GEMV, fused, fp32 operand
    (1, 512, "bf16", "f32"),     # streaming GEMV, fused, H = 512
    (5, 1024, "bf16", "bf16"),   # tile kernel, fused
    (64, 1024, "f32", "bf16"),   # tile kernel, fused, f32 input
    (70, 1024, "bf16", "bf16"),  # blocked GEMM, prologue kernel
    (82, 1024, "bf16", "f32"),   # fp32 operand, 65-128 rows: narrow GEMM + tile pass + GEMV, prologue kernel
    (8, 1024, "bf16", "f32"),    # exact-split MFMA path, prologue kernel
    (4, 40, "f16", "f32"),       # generic path, prologue kernel
])
def test_prenorm_greedy(batch, H, hidden_dtype, act_dtype):
    rng = np.random.default_rng(batch * 7 + H)
    V = 4099
    x, nw, W = _inputs(rng, batch, H, V, hidden_dtype)
    ids = nvjsel.lm_head_greedy_top1_hip(
        torch.from_numpy(x).to(TORCH[hidden_dtype]).cuda(), torch.from_numpy(W).to(torch.bfloat16).cuda(),
        weight_layout="vh", norm_weight=torch.from_numpy(nw).cuda(), rms_norm_eps=1e-6,
        act_dtype=TORCH[act_dtype])
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype=hidden_dtype, act_dtype=act_dtype)
    z = sel.lm_head_logits(xin, W)
    check_greedy(ids.cpu().numpy(), z, RC.get((act_dtype, "bf16"), 0),
                 f"prenorm B={batch} H={H} {hidden_dtype}->{act_dtype}")


@pytest.mark.parametrize("batch,hidden_dtype,act_dtype", [
    (12, "bf16", "bf16"),  # tile kernel, hidden one element past a 16-byte boundary: element loads
    (40, "f16", "bf16"),   # tile kernel, f16 hidden: 16-byte loads converted per element
    (7, "bf16", "f32"),    # tile kernel, three-term activations from an unaligned bf16 hidden
])
def test_prenorm_tile_unaligned_and_f16_hidden(batch, hidden_dtype, act_dtype):
    """The tile kernel's prologue loads a 16-byte-aligned bf16 hidden straight
    into its fragment registers and any other hidden eight elements at a time
    (16-byte loads when aligned, element loads when not)."""
    rng = np.random.default_rng(500 + batch)
    H, V = 1024, 5003
    x, nw, W = _inputs(rng, batch, H, V, hidden_dtype)
    xt = torch.from_numpy(x).to(TORCH[hidden_dtype]).cuda()
    if hidden_dtype == "bf16":  # the same rows one element into a buffer: an unaligned base pointer
        buf = torch.zeros(batch * H + 1, dtype=xt.dtype, device="cuda")
        buf[1:] = xt.reshape(-1)
        xt = buf[1:].view(batch, H)
        assert xt.data_ptr() % 16 != 0
    ids = nvjsel.lm_head_greedy_top1_hip(
        xt, torch.from_numpy(W).to(torch.bfloat16).cuda(), weight_layout="vh",
        norm_weight=torch.from_numpy(nw).cuda(), rms_norm_eps=1e-6, act_dtype=TORCH[act_dtype])
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype=hidden_dtype, act_dtype=act_dtype)
    z = sel.lm_head_logits(xin, W)
    check_greedy(ids.cpu().numpy(), z, RC.get((act_dtype, "bf16"), 0),
                 f"prenorm tile B={batch} {hidden_dtype}->{act_dtype}")


@pytest.mark.parametrize("batch,act_dtype", [(1, "bf16"), (2, "f32"), (16, "bf16"), (24, "bf16"), (64, "bf16"), (9, "f32"),
                                             (90, "f32"), (110, "f32")])
def test_prenorm_fused_sample(batch, act_dtype):
    rng = np.random.default_rng(300 + batch)
    H, V = 1024, 8191
    x, nw, W = _inputs(rng, batch, H, V, "bf16")
    temps = np.where(np.arange(batch) % 3 == 0, 0.0, 0.8).astype(np.float32)
    keys = engine_keys(batch, 11)
    ids = nvjsel.lm_head_sample_token_ids(
        torch.from_numpy(x).to(torch.bfloat16).cuda(), torch.from_numpy(W).to(torch.bfloat16).cuda(),
        temperatures=torch.from_numpy(temps).cuda(), rng_keys=keys_tensor(keys), weight_layout="vh",
        norm_weight=torch.from_numpy(nw).cuda(), act_dtype=TORCH[act_dtype])
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype="bf16", act_dtype=act_dtype)
    z = sel.lm_head_logits(xin, W)
    check_fused_sampled(ids.cpu().numpy(), z, temps, keys, RC.get((act_dtype, "bf16"), 0), f"B={batch}")


@pytest.mark.parametrize("hidden_dtype,act_dtype", [("bf16", "bf16"), ("f32", "f32"), ("f16", "bf16")])
def test_rms_norm_tensor(hidden_dtype, act_dtype):
    """nvjsel.rms_norm_hip against the oracle: exact but for one rounding step
    of the activation type (the mean of squares is summed in another order)."""
    rng = np.random.default_rng(5)
    x, nw, _ = _inputs(rng, 6, 1024, 16, hidden_dtype)
    got = nvjsel.rms_norm_hip(torch.from_numpy(x).to(TORCH[hidden_dtype]).cuda(), torch.from_numpy(nw).cuda(),
                              1e-6, TORCH[act_dtype]).float().cpu().numpy()
    exp = sel.lm_head_input(x, nw, 1e-6, hidden_dtype=hidden_dtype, act_dtype=act_dtype)
    ulp = {"f32": 2.0 ** -23, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}[act_dtype]
    diff = np.abs(got.astype(np.float64) - exp)
    assert np.all(diff <= np.abs(exp) * ulp * 2 + 1e-30)
    if act_dtype != "f32":  # a last-place change of the fp32 value rarely moves the rounded one
        assert np.mean(diff == 0) > 0.95


def test_prenorm_topk_route_uses_normed_logits():
    """With top_k the pre-norm route normalises, forms logits and samples: with
    top_k = 1 that is the greedy answer of the normed operand."""
    rng = np.random.default_rng(9)
    x, nw, W = _inputs(rng, 3, 1024, 4099, "bf16")
    ids = nvjsel.lm_head_sample_token_ids(
        torch.from_numpy(x).to(torch.bfloat16).cuda(), torch.from_numpy(W).to(torch.bfloat16).cuda(),
        temperatures=torch.ones(3).cuda(), rng_keys=keys_tensor(engine_keys(3, 0)),
        top_k=torch.ones(3, dtype=torch.int32).cuda(), weight_layout="vh",
        norm_weight=torch.from_numpy(nw).cuda(), act_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    xin = sel.lm_head_input(x, nw, 1e-6, hidden_dtype="bf16", act_dtype="bf16")
    check_greedy(ids.cpu().numpy(), sel.lm_head_logits(xin, W), 1, "top_k=1")


def test_prenorm_rejects_bad_norm_weight():
    x = torch.zeros(2, 1024, dtype=torch.bfloat16).cuda()
    W = torch.zeros(64, 1024, dtype=torch.bfloat16).cuda()
    with pytest.raises(ValueError, match="norm_weight"):
        nvjsel.lm_head_greedy_top1_hip(x, W, weight_layout="vh", norm_weight=torch.zeros(512).cuda())


def test_workspace_reuse_across_prologue_paths():
    """A prologue-kernel call leaves its rows in the shared workspace zeroed
    again, so a later call of another shape finds its accumulators at rest."""
    rng = np.random.default_rng(21)
    W = sel.round_bf16(rng.normal(0.0, 0.02, (4099, 1024)).astype(np.float32))
    Wt = torch.from_numpy(W).to(torch.bfloat16).cuda()
    nw = rng.normal(0.0, 0.2, 1024).astype(np.float32)
    for batch, act in [(8, "f32"), (64, "bf16"), (3, "f32"), (33, "bf16"), (1, "bf16")]:
        x = sel.round_bf16(rng.normal(0.0, 3.0, (batch, 1024)).astype(np.float32))
        ids = nvjsel.lm_head_greedy_top1_hip(torch.from_numpy(x).to(torch.bfloat16).cuda(), Wt, weight_layout="vh",
                                             norm_weight=torch.from_numpy(nw).cuda(), act_dtype=TORCH[act])
        torch.cuda.synchronize()
        z = sel.lm_head_logits(sel.lm_head_input(x, nw, 1e-6, hidden_dtype="bf16", act_dtype=act), W)
        check_greedy(ids.cpu().numpy(), z, RC.get((act, "bf16"), 0), f"reuse B={batch}")
