"""C-ABI checks that need no GPU: the library loads, exports every entry point
include/nvjsel.h declares, and rejects bad arguments before any launch."""
import ctypes
import re
from pathlib import Path

import pytest

from nvjsel import _lib
from nvjsel import registry

HEADER = Path(__file__).resolve().parents[1] / "include" / "nvjsel.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nvjsel_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_functions() == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_functions():
        getattr(raw, name)  # raises AttributeError if not exported
    assert lib.nvjsel_abi_version() == _lib.ABI_VERSION


def test_workspace_sizes():
    lib = _lib.load()
    assert lib.nvjsel_lm_head_workspace_size(0) == 0
    assert lib.nvjsel_lm_head_workspace_size(1) >= 8
    assert lib.nvjsel_lm_head_workspace_size(256) >= 256 * 8
    assert lib.nvjsel_sample_workspace_size(256, 248320) >= 256 * 16


DUMMY = 0x1000  # never dereferenced: validation fails first


@pytest.mark.parametrize("args,code", [
    # batch 0
    ((DUMMY, 1, DUMMY, 1, 0, 0, 32, 257, 1, DUMMY, None, DUMMY, 4096, None), -1),
    # bad dtype
    ((DUMMY, 7, DUMMY, 1, 0, 1, 32, 257, 1, DUMMY, None, DUMMY, 4096, None), -1),
    # bad layout
    ((DUMMY, 1, DUMMY, 1, 5, 1, 32, 257, 1, DUMMY, None, DUMMY, 4096, None), -1),
    # bad reduce_cast
    ((DUMMY, 1, DUMMY, 1, 0, 1, 32, 257, 9, DUMMY, None, DUMMY, 4096, None), -1),
    # null hidden
    ((None, 1, DUMMY, 1, 0, 1, 32, 257, 1, DUMMY, None, DUMMY, 4096, None), -1),
    # workspace too small
    ((DUMMY, 1, DUMMY, 1, 0, 64, 32, 257, 1, DUMMY, None, DUMMY, 8, None), -3),
])
def test_lm_head_top1_validation(args, code):
    lib = _lib.load()
    assert lib.nvjsel_lm_head_top1(*args) == code
    assert lib.nvjsel_last_error()


def test_sample_validation():
    lib = _lib.load()
    assert lib.nvjsel_sample(None, 0, 4, 100, 100, DUMMY, None, None, DUMMY, None, DUMMY, DUMMY, 4096, None) == -1
    assert lib.nvjsel_sample(DUMMY, 0, 4, 100, 50, DUMMY, None, None, DUMMY, None, DUMMY, DUMMY, 4096, None) == -1
    assert lib.nvjsel_sample(DUMMY, 3, 4, 100, 100, DUMMY, None, None, DUMMY, None, DUMMY, DUMMY, 4096, None) == -1
    assert lib.nvjsel_sample(DUMMY, 0, 4, 100, 100, DUMMY, None, None, DUMMY, None, DUMMY, DUMMY, 1, None) == -3
    assert lib.nvjsel_lm_head_sample(DUMMY, 1, DUMMY, 1, 0, 2, 32, 10, 1, None, DUMMY, DUMMY, DUMMY, 4096, None) == -1
    assert lib.nvjsel_derive_keys(DUMMY, DUMMY, 0, DUMMY, None, None) == -1
    with pytest.raises(_lib.NvjselError) as ei:
        _lib.call("nvjsel_derive_keys", None, None, 3, None, None, None)
    assert "null" in str(ei.value)


def test_registry_semantics():
    assert registry.lm_head_greedy_top1_impl(None) == "jax"
    assert registry.lm_head_greedy_top1_impl("Triton") == "triton"
    assert registry.lm_head_greedy_top1_impl("fused_gemm") == "cutlass"
    assert registry.lm_head_greedy_top1_impl("hip") == "hip"
    with pytest.raises(ValueError):
        registry.lm_head_greedy_top1_impl("bogus")
    st = registry.select_token_selection_backend("auto")
    assert st.selected == "hip" and st.available
    # the reference's status record, field for field (kernels/registry.py:30-52)
    assert list(st.as_dict()) == ["requested", "selected", "available", "implemented", "external_kernels_enabled",
                                  "missing_modules", "provided_kernels", "fallback", "reason"]
    assert st.implemented and st.external_kernels_enabled and st.fallback is None and st.missing_modules == ()
    with pytest.raises(ValueError):
        registry.select_token_selection_backend("nope")


def test_registry_strict_raises_when_library_missing(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(registry.KernelBackendUnavailable):
        registry.select_token_selection_backend("hip")
    st = registry.select_token_selection_backend("hip", strict=False)
    assert not st.available and not st.external_kernels_enabled and st.missing_modules == ("missing.so",)
    assert st.fallback is None  # never a silent fallback


def test_host_api_rejects_bad_shapes_before_launch():
    torch = pytest.importorskip("torch")
    import nvjsel

    h = torch.zeros(3, 2, 32, dtype=torch.bfloat16)
    w = torch.zeros(32, 257, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"\[B, 1, H\]"):
        nvjsel.lm_head_greedy_top1_hip(h, w)
    with pytest.raises(ValueError, match="must match"):
        nvjsel.lm_head_greedy_top1_hip(torch.zeros(3, 1, 16, dtype=torch.bfloat16), w)
    with pytest.raises(ValueError, match="dtype"):
        nvjsel.lm_head_greedy_top1_hip(torch.zeros(3, 1, 32, dtype=torch.int8), w)
    with pytest.raises(ValueError, match="device"):
        nvjsel.lm_head_greedy_top1_hip(torch.zeros(3, 1, 32, dtype=torch.bfloat16), w)
    with pytest.raises(ValueError, match="non-empty"):
        nvjsel.lm_head_greedy_top1_hip(torch.zeros(0, 1, 32, dtype=torch.bfloat16), w)


def test_product_code_never_imports_the_oracle():
    """The oracle is the checker only: the package and bench's GPU path do not use it."""
    root = Path(__file__).resolve().parents[1]
    for f in list((root / "nano-vllm-jax_amd").rglob("*.py")) + list((root / "nano-vllm-jax_amd").rglob("*.hip")):
        assert "oracle" not in f.read_text(), f
    # bench.py imports the oracle only inside its CPU-baseline functions (cpu_*)
    import ast

    tree = ast.parse((root / "bench.py").read_text())
    allowed = set()
    for fn in ast.walk(tree):
        if isinstance(fn, ast.FunctionDef) and fn.name.startswith("cpu_"):
            allowed.update(id(n) for n in ast.walk(fn))
    for node in ast.walk(tree):
        if isinstance(node, (ast.Import, ast.ImportFrom)):
            names = [a.name for a in node.names] + ([node.module] if isinstance(node, ast.ImportFrom) else [])
            if any(n and n.split(".")[0] == "oracle" for n in names):
                assert id(node) in allowed, f"bench.py line {node.lineno} imports the oracle outside cpu_*"


def test_mtp_registry_and_shape_contract():
    assert registry.mtp_lm_head_greedy_top1_impl(None) == "jax"
    assert registry.mtp_lm_head_greedy_top1_impl("triton_top1") == "triton"
    assert registry.mtp_lm_head_greedy_top1_impl("fused_gemm") == "cutlass"
    assert registry.mtp_lm_head_greedy_top1_impl("HIP") == "hip"
    with pytest.raises(ValueError):
        registry.mtp_lm_head_greedy_top1_impl("bogus")
    torch = pytest.importorskip("torch")
    import nvjsel
    with pytest.raises(ValueError, match=r"\[B, T, H\]"):
        nvjsel.mtp_greedy_top1_token_ids(torch.zeros(2, 8), torch.zeros(16, 8, dtype=torch.bfloat16))


def test_bench_refuses_more_than_one_gpu():
    """Every box has one GPU: bench.py --gpus N > 1 exits with a JSON message
    (status 2) before touching a device."""
    import json
    import subprocess
    import sys

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert msg["n_gpus"] == 2 and "one GPU" in msg["error"]


def test_bench_timed_regions_hold_exactly_steps_calls():
    """bench.time_config: the warmup steps and the settle phase run untimed
    before the timed regions, and each timed region holds exactly `steps`
    calls between two device synchronisations (a stand-in device that only
    records the call order)."""
    import sys
    import time

    root = Path(__file__).resolve().parents[1]
    sys.path.insert(0, str(root))
    import bench

    log = []

    class Event:
        def __init__(self, enable_timing=False):
            self.t = None

        def record(self):
            log.append("event")
            self.t = time.perf_counter()

        def elapsed_time(self, other):
            return (other.t - self.t) * 1e3

    from types import SimpleNamespace

    FakeTorch = SimpleNamespace(cuda=SimpleNamespace(Event=Event, synchronize=lambda: log.append("sync")))

    class Cfg:
        def launch(self, i):
            log.append(("call", i))

    med, p90, ms = bench.time_config(FakeTorch, Cfg(), steps=7, warmup=3, repeats=4, ncopies=2, settle_s=0.01)
    assert len(ms) == 4 and med <= p90
    first_event = log.index("event")
    untimed = [e for e in log[:first_event] if e != "sync"]
    assert len(untimed) >= 3 + 10  # the warmup steps, then at least one settle round of ten calls
    assert [e[1] for e in untimed[:3]] == [0, 1, 0]
    # the timed part: per region sync, event, exactly 7 calls, event, sync
    timed = log[first_event - 1:]
    for r in range(4):
        region = timed[r * 11:(r + 1) * 11]
        assert region[0] == "sync" and region[1] == "event" and region[9] == "event" and region[10] == "sync"
        assert [e[1] for e in region[2:9]] == [s % 2 for s in range(7)]
    assert len(timed) == 44
