"""GPU: the allocation-free greedy LM-head entry point against the regular one.

nvjsel_lm_head_top1_noalloc keeps its workspace in a fixed device array
instead of a caller workspace; its ids (and winning logits) must equal
nvjsel_lm_head_top1's on the same inputs -- on two calls in a row, the second
with a smaller batch (the array keeps the first call's state between calls),
across the streaming (B <= 2), tile (3..64), blocked-GEMM (65..256) and
multi-pass (> 256: 256-row passes reusing the keys and ticket) paths."""
import numpy as np
import pytest
import torch

from nvjsel import _lib

pytestmark = pytest.mark.gpu

def _noalloc(lib):
    return lib.nvjsel_lm_head_top1_noalloc  # argtypes from nvjsel._lib.SIGNATURES


def _run_both(lib, h, W, B, H, V):
    stream = torch.cuda.current_stream().cuda_stream
    ids_a = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    best_a = torch.zeros(B, dtype=torch.float32, device="cuda")
    ws = torch.zeros(lib.nvjsel_lm_head_workspace_size(B), dtype=torch.uint8, device="cuda")
    _lib.call("nvjsel_lm_head_top1", h.data_ptr(), _lib.BF16, W.data_ptr(), _lib.BF16, _lib.W_VH, B, H, V, 1,
              ids_a.data_ptr(), best_a.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    ids_b = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    best_b = torch.zeros(B, dtype=torch.float32, device="cuda")
    rc = _noalloc(lib)(h.data_ptr(), _lib.BF16, W.data_ptr(), _lib.BF16, _lib.W_VH, B, H, V, 1, ids_b.data_ptr(),
                       best_b.data_ptr(), stream)
    assert rc == 0, lib.nvjsel_last_error()
    torch.cuda.synchronize()
    return ids_a.cpu().numpy(), best_a.cpu().numpy(), ids_b.cpu().numpy(), best_b.cpu().numpy()


@pytest.mark.parametrize("batches", [(64, 8), (1, 1), (200, 2), (33, 3), (300, 70)])
def test_noalloc_matches_workspace_entry(batches):
    lib = _lib.load()
    rng = np.random.default_rng(sum(batches))
    H, V = 1024, 50_000
    W = torch.from_numpy(rng.standard_normal((V, H)).astype(np.float32) * 0.02).cuda().to(torch.bfloat16)
    for B in batches:  # second call smaller
        h = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda().to(torch.bfloat16)
        ia, ba, ib, bb = _run_both(lib, h, W, B, H, V)
        assert np.array_equal(ia, ib), (B, ia[:8], ib[:8])
        assert np.array_equal(ba.view(np.uint32), bb.view(np.uint32)), B
        assert np.all((ia >= 0) & (ia < V))


def test_noalloc_hv_weights():
    """[H, V] weights through the no-alloc entry: the streaming kernel (8
    rows) and the blocked GEMM with transposing reads (40 rows), on two calls
    in a row, against the workspace entry."""
    lib = _lib.load()
    rng = np.random.default_rng(77)
    H, V = 1024, 20008
    Whv = torch.from_numpy(rng.standard_normal((H, V)).astype(np.float32) * 0.02).cuda().to(torch.bfloat16)
    stream = torch.cuda.current_stream().cuda_stream
    for B in (40, 8):  # second call smaller
        h = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda().to(torch.bfloat16)
        ids_a = torch.full((B,), -1, dtype=torch.int32, device="cuda")
        ws = torch.zeros(lib.nvjsel_lm_head_workspace_size(B), dtype=torch.uint8, device="cuda")
        _lib.call("nvjsel_lm_head_top1", h.data_ptr(), _lib.BF16, Whv.data_ptr(), _lib.BF16, _lib.W_HV, B, H, V, 1,
                  ids_a.data_ptr(), None, ws.data_ptr(), ws.numel(), stream)
        ids_b = torch.full((B,), -1, dtype=torch.int32, device="cuda")
        rc = _noalloc(lib)(h.data_ptr(), _lib.BF16, Whv.data_ptr(), _lib.BF16, _lib.W_HV, B, H, V, 1,
                           ids_b.data_ptr(), None, stream)
        assert rc == 0, lib.nvjsel_last_error()
        torch.cuda.synchronize()
        assert torch.equal(ids_a, ids_b), B
        assert bool(((ids_a >= 0) & (ids_a < V)).all())


def test_noalloc_rejects_batch_beyond_scratch():
    lib = _lib.load()
    rc = _noalloc(lib)(0x1000, _lib.BF16, 0x1000, _lib.BF16, _lib.W_VH, 4097, 1024, 1000, 1, 0x1000, None, None)
    assert rc == -2
    assert b"4096" in lib.nvjsel_last_error()


_CAPTURE_SCRIPT = r"""
import sys, numpy as np, torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/nano-vllm-jax_amd")
from nvjsel import _lib
lib = _lib.load()
rng = np.random.default_rng(5)
B, H, V = 8, 1024, 30_000
W = torch.from_numpy(rng.standard_normal((V, H)).astype(np.float32) * 0.02).cuda().to(torch.bfloat16)
hs = [torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda().to(torch.bfloat16) for _ in range(3)]
h = hs[0].clone()
ids = torch.full((B,), -1, dtype=torch.int32, device="cuda")
s = torch.cuda.Stream()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    # the process's first no-alloc call: the scratch address is looked up
    # here, under capture; nothing but the LM-head kernels is recorded
    rc = lib.nvjsel_lm_head_top1_noalloc(h.data_ptr(), _lib.BF16, W.data_ptr(), _lib.BF16, _lib.W_VH, B, H, V, 1,
                                         ids.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.nvjsel_last_error()
ws = torch.zeros(lib.nvjsel_lm_head_workspace_size(B), dtype=torch.uint8, device="cuda")
for rep in range(6):
    h.copy_(hs[rep % 3])
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    ref = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    _lib.call("nvjsel_lm_head_top1", h.data_ptr(), _lib.BF16, W.data_ptr(), _lib.BF16, _lib.W_VH, B, H, V, 1,
              ref.data_ptr(), None, ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(ids, ref), (rep, ids.tolist(), ref.tolist())
print("capture ok")
"""


def test_noalloc_first_call_under_graph_capture(tmp_path):
    """A fresh process whose FIRST no-alloc call is made under HIP graph
    capture: the scratch array must already be zero (no fill is recorded),
    and every replay -- with the process's own eager calls between them --
    must equal the workspace entry point's ids."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    script = tmp_path / "capture_first_call.py"
    script.write_text(_CAPTURE_SCRIPT)
    r = subprocess.run([sys.executable, str(script), root], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "capture ok" in r.stdout
