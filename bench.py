"""Benchmark of decode-step token selection on one MI355X.

Prints ONE JSON line.  The headline workload (``value``) is BASELINE config 0:
greedy LM-head top-1 at B=1, V=248320, H=1024, bf16 -- the configuration the
metric's HBM-roofline target is quoted on.  The other four BASELINE configs
(temperature sampling B=8, top-k/top-p B=64, fused LM-head + Gumbel B=64,
mixed per-row parameters B=256) are timed in the same run and reported under
``per_config``.  Inputs are synthetic, seeded, and resident in HBM before the
timed region; each step is one call of the C ABI on torch's current stream.

``cpu_baseline`` times the numpy oracle (fp32 matmul + argmax) for config 0 on
the host cores, on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "nano-vllm-jax_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK = 8.0e12  # bytes/s, MI355X
V_FULL, H_FULL = 248320, 1024


def _parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5,x1,x2")
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="bounded CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 512 MiB device copy (rocprofv3 counter calibration)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "lm_head_gemv_c1_traffic.txt")


def committed_traffic():
    """HBM bytes per launch of the C1 kernel from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def calibrate_copy(torch):
    n = 512 * 1024 * 1024
    src = torch.ones(n // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": n}))


class Cfg:
    """One BASELINE config: device inputs + a launch closure + algorithmic bytes."""

    def __init__(self, name, batch, nbytes, launch, kernel, desc):
        self.name, self.batch, self.nbytes, self.launch, self.kernel, self.desc = (
            name, batch, nbytes, launch, kernel, desc)


def _zipf_rows(torch, gen, batch, vocab, s_lo, s_hi, noise_sd, dev):
    ranks = torch.arange(1, vocab + 1, device=dev, dtype=torch.float32)
    s = s_lo + (s_hi - s_lo) * torch.rand(batch, 1, device=dev, generator=gen)
    lp = -s * torch.log(ranks)[None, :]
    lp = lp - torch.logsumexp(lp, dim=1, keepdim=True)
    perm = torch.argsort(torch.rand(batch, vocab, device=dev, generator=gen), dim=1)
    lp = torch.gather(lp, 1, perm)
    return lp + noise_sd * torch.randn(batch, vocab, device=dev, generator=gen)


def build_configs(torch, which):
    import numpy as np

    from nvjsel import _lib

    lib = _lib.load()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    stream = lambda: torch.cuda.current_stream(dev).cuda_stream  # noqa: E731
    cfgs = []
    W = None

    def weights():
        nonlocal W
        if W is None:
            # two copies, alternated per step, so the 508 MB table cannot sit in the 256 MB MALL
            W = [(torch.randn(V_FULL, H_FULL, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
                 for _ in range(2)]
        return W

    def keys_for(batch, row_seed=False):
        if row_seed:  # PRNGKey(seed) = (0, seed) for 32-bit seeds
            k = np.stack([np.zeros(batch, np.uint32), np.arange(batch, dtype=np.uint32)], axis=1)
            return torch.from_numpy(k.view(np.int32).copy()).to(dev)
        # the executor's keys fold_in(fold_in(PRNGKey(0), slot), counter), derived on device
        from nvjsel import derive_rng_keys

        keys, _ = derive_rng_keys(torch.arange(batch, dtype=torch.int32, device=dev),
                                  torch.zeros(batch, dtype=torch.int32, device=dev))
        return keys

    def ws(nbytes):
        return torch.zeros(max(int(nbytes), 4096), dtype=torch.uint8, device=dev)

    if "c1" in which:
        Ws = weights()
        h = torch.randn(1, H_FULL, device=dev, generator=gen).to(torch.bfloat16)
        out = torch.empty(1, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_lm_head_workspace_size(1))
        state = {"i": 0}

        def launch(Ws=Ws, h=h, out=out, w=w, state=state):
            Wi = Ws[state["i"] & 1]
            state["i"] += 1
            rc = lib.nvjsel_lm_head_top1(h.data_ptr(), 1, Wi.data_ptr(), 1, 0, 1, H_FULL, V_FULL, 1,
                                         out.data_ptr(), None, w.data_ptr(), w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("c1_greedy_lm_head_b1", 1, V_FULL * H_FULL * 2 + H_FULL * 2, launch,
                        "lm_head_gemv_kernel", "greedy LM-head top-1, B=1, bf16 W[248320,1024]"))

    if "c2" in which:
        B = 8
        l = torch.randn(B, V_FULL, device=dev, generator=gen) * 3
        for b in range(B):
            idx = torch.randperm(V_FULL, device=dev, generator=gen)[:5]
            l[b, idx] += 12.0
        t = torch.full((B,), 0.7, device=dev)
        keys = keys_for(B, row_seed=True)
        out = torch.empty(B, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_sample_workspace_size(B, V_FULL))

        def launch(l=l, t=t, keys=keys, out=out, w=w, B=B):
            rc = lib.nvjsel_sample(l.data_ptr(), 0, B, V_FULL, V_FULL, t.data_ptr(), None, None,
                                   keys.data_ptr(), None, out.data_ptr(), w.data_ptr(), w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("c2_temperature_b8", B, B * V_FULL * 4, launch, "sample_onepass_kernel",
                        "temperature sampling, f32 logits [8,248320], T=0.7"))

    if "c3" in which:
        B = 64
        l = _zipf_rows(torch, gen, B, V_FULL, 1.1, 1.1, 0.5, dev).float().contiguous()
        t = torch.full((B,), 0.8, device=dev)
        k = torch.full((B,), 50, dtype=torch.int32, device=dev)
        p = torch.full((B,), 0.9, device=dev)
        keys = keys_for(B)
        out = torch.empty(B, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_sample_workspace_size(B, V_FULL))

        def launch(l=l, t=t, k=k, p=p, keys=keys, out=out, w=w, B=B):
            rc = lib.nvjsel_sample(l.data_ptr(), 0, B, V_FULL, V_FULL, t.data_ptr(), k.data_ptr(),
                                   p.data_ptr(), keys.data_ptr(), None, out.data_ptr(), w.data_ptr(),
                                   w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("c3_topk_topp_b64", B, B * V_FULL * 4, launch, "sample_select_kernel",
                        "top-k=50 / top-p=0.9 / T=0.8, f32 logits [64,248320] Zipf(1.1)"))

    if "c4" in which:
        B = 64
        Ws = weights()
        h = torch.randn(B, H_FULL, device=dev, generator=gen).to(torch.bfloat16)
        t = torch.ones(B, device=dev)
        keys = keys_for(B)
        out = torch.empty(B, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_lm_head_workspace_size(B))
        state = {"i": 0}

        def launch(h=h, t=t, keys=keys, out=out, w=w, B=B, Ws=Ws, state=state):
            Wi = Ws[state["i"] & 1]
            state["i"] += 1
            rc = lib.nvjsel_lm_head_sample(h.data_ptr(), 1, Wi.data_ptr(), 1, 0, B, H_FULL, V_FULL, 1,
                                           t.data_ptr(), keys.data_ptr(), out.data_ptr(), w.data_ptr(),
                                           w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("c4_fused_lm_head_gumbel_b64", B, V_FULL * H_FULL * 2 + B * H_FULL * 2, launch,
                        "lm_head_tile_kernel", "fused LM-head + Gumbel-max, B=64, T=1"))

    if "c5" in which:
        B = 256
        l = _zipf_rows(torch, gen, B, V_FULL, 1.05, 1.3, 1.0, dev).to(torch.bfloat16).contiguous()
        choice = lambda vals, dt: torch.tensor(vals, device=dev, dtype=dt)[  # noqa: E731
            torch.randint(0, len(vals), (B,), device=dev, generator=gen)]
        t = choice([0.0, 0.6, 1.0], torch.float32)
        k = choice([0, 20, 100], torch.int32)
        p = choice([1.0, 0.95, 0.8], torch.float32)
        keys = keys_for(B)
        out = torch.empty(B, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_sample_workspace_size(B, V_FULL))

        def launch(l=l, t=t, k=k, p=p, keys=keys, out=out, w=w, B=B):
            rc = lib.nvjsel_sample(l.data_ptr(), 1, B, V_FULL, V_FULL, t.data_ptr(), k.data_ptr(),
                                   p.data_ptr(), keys.data_ptr(), None, out.data_ptr(), w.data_ptr(),
                                   w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("c5_mixed_b256_bf16", B, B * V_FULL * 2, launch, "sample_gumbel_kernel",
                        "mixed per-row T/top-k/top-p, bf16 logits [256,248320]"))
    if "x1" in which:  # the final-RMSNorm prologue fused into the C1 launch
        Ws = weights()
        h = (torch.randn(1, H_FULL, device=dev, generator=gen) * 4).to(torch.bfloat16)
        nw = (torch.randn(H_FULL, device=dev, generator=gen) * 0.1).float()
        out = torch.empty(1, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_lm_head_prenorm_workspace_size(1, H_FULL))
        state = {"i": 0}

        def launch(Ws=Ws, h=h, nw=nw, out=out, w=w, state=state):
            Wi = Ws[state["i"] & 1]
            state["i"] += 1
            rc = lib.nvjsel_lm_head_top1_prenorm(h.data_ptr(), 1, nw.data_ptr(), 0, 1e-6, 1, Wi.data_ptr(), 1, 0,
                                                 1, H_FULL, V_FULL, 1, out.data_ptr(), None, w.data_ptr(),
                                                 w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("x1_prenorm_greedy_lm_head_b1", 1, V_FULL * H_FULL * 2 + H_FULL * 2, launch,
                        "lm_head_gemv_kernel", "C1 with the final RMSNorm applied in the launch (bf16 act)"))

    if "x2" in which:  # top-k values/indices of the verifier route on the C3 logits shape
        B, K = 64, 50
        l = _zipf_rows(torch, gen, B, V_FULL, 1.1, 1.1, 0.5, dev).float().contiguous()
        vals = torch.empty(B, K, dtype=torch.float32, device=dev)
        idx = torch.empty(B, K, dtype=torch.int32, device=dev)
        w = ws(lib.nvjsel_topk_workspace_size(B, V_FULL))

        def launch(l=l, vals=vals, idx=idx, w=w, B=B, K=K):
            rc = lib.nvjsel_topk(l.data_ptr(), 0, B, V_FULL, V_FULL, K, vals.data_ptr(), idx.data_ptr(),
                                 w.data_ptr(), w.numel(), stream())
            assert rc == 0, lib.nvjsel_last_error()

        cfgs.append(Cfg("x2_topk50_b64", B, B * V_FULL * 4, launch, "topk_select_kernel",
                        "top-k values+indices k=50, f32 logits [64,248320] Zipf(1.1)"))
    torch.cuda.synchronize()
    return cfgs


def time_config(torch, cfg, steps, warmup):
    for _ in range(warmup):
        cfg.launch()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        cfg.launch()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    return ms


def cpu_baseline_c1(seconds):
    """numpy oracle for config 0 (fp32 matmul + argmax) on the host cores."""
    import numpy as np

    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    h = rng.standard_normal((1, H_FULL)).astype(np.float32)
    W = (rng.standard_normal((V_FULL, H_FULL), dtype=np.float32) * 0.02)
    np.argmax(h @ W.T, axis=1)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        np.argmax(h @ W.T, axis=1)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / n
    return {"value": 1.0 / per, "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "sample": f"{n} calls of numpy fp32 [1,1024]x[1024,248320] matmul + argmax "
                      f"({el:.1f} s); threads = BLAS pool size",
            "ms_per_call": per * 1e3}


def main():
    args = _parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; the multi-GPU (vocab-sharded) "
                                   "path is design-only", "n_gpus": args.gpus}))
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    which = set(args.configs.split(","))
    which.add("c1")
    cfgs = build_configs(torch, which)
    per = {}
    for cfg in cfgs:
        ms = time_config(torch, cfg, args.steps, args.warmup)
        us = ms * 1e3
        per[cfg.name] = {
            "desc": cfg.desc,
            "us_per_step": round(us, 3),
            "tokens_per_s": round(cfg.batch / (ms * 1e-3), 1),
            "hbm_bytes_per_step": cfg.nbytes,
            "hbm_frac": round(cfg.nbytes / (ms * 1e-3) / HBM_PEAK, 4),
            "dominant_kernel": cfg.kernel,
        }
        print(f"# {cfg.name}: {us:.2f} us/step, {per[cfg.name]['tokens_per_s']:.0f} tok/s, "
              f"{per[cfg.name]['hbm_frac'] * 100:.1f}% of HBM peak", file=sys.stderr, flush=True)
    head = per["c1_greedy_lm_head_b1"]
    ms_head = head["us_per_step"] / 1e3
    achieved = head["hbm_bytes_per_step"] / (ms_head * 1e-3)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_c1(args.cpu_seconds)
    line = {
        "metric": "sampled tokens/s at B=1,64,256 (V=248k) + % of 8 TB/s HBM roofline",
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_head, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch RNG on device; random-init weights)",
        "config": {"workload": "c1_greedy_lm_head_b1: greedy LM-head top-1, hidden [1,1024] bf16 x "
                               "W [248320,1024] bf16, fp32 accumulate, bf16-rounded logits",
                   "batch": 1, "vocab": V_FULL, "hidden": H_FULL},
        "roofline": {"bound": "hbm", "achieved": round(achieved / 1e9, 1), "peak": HBM_PEAK / 1e9,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK, 4), "traffic": committed_traffic()},
        "cpu_baseline": cpu,
        "per_config": per,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
