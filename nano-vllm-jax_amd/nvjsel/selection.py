"""Host-side mirror of the reference's token-selection interface, on torch-ROCm.

Device memory and streams come from torch; every computation runs in
libnvjsel.so (HIP, gfx950) through the C ABI of include/nvjsel.h.

Mirrors:
* ``lm_head_greedy_top1_hip``  <- ``lm_head_greedy_top1_triton``
  (nanovllm_jax/kernels/lm_head_triton.py:114-186): same argument meaning,
  same ``ValueError`` checks, returns int32 ``[B, 1]``.
* ``lm_head_sample_token_ids`` <- ``lm_head_sample_token_ids``
  (nanovllm_jax/model.py:901-938): ``T <= 0`` rows greedy, others
  ``categorical(key, logits / max(T, 1e-6))``; extended with optional per-row
  ``top_k`` / ``top_p`` (docs/kernel_roadmap.md:436-439).
* ``sample_token_ids``         <- the roadmap ABI
  ``sample_topk_topp(logits, temperature, top_k, top_p, rng_state) -> token_ids``.
* ``derive_rng_keys``          <- the executor's key derivation
  (nanovllm_jax/engine/model_executor.py:2131, 2214-2219, 2231).
"""
from __future__ import annotations

import threading

import torch

from . import _lib

_TORCH_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _TORCH_DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported {what} dtype: {t.dtype}") from None


def _require_cuda(*ts: torch.Tensor) -> torch.device:
    dev = ts[0].device
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("nvjsel kernels take device tensors (got a CPU tensor)")
        if t.device != dev:
            raise ValueError("all tensors must live on one device")
    return dev


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


class _WorkspacePool:
    """Zero-filled scratch buffers per (device, stream, kind).

    Each entry point leaves its workspace zero-filled when it returns, so a
    buffer is zeroed once at allocation and reused in stream order."""

    def __init__(self):
        self._bufs: dict = {}
        self._lock = threading.Lock()

    def get(self, device: torch.device, stream: int, kind: str, nbytes: int) -> torch.Tensor:
        key = (device.index, stream, kind)
        with self._lock:
            buf = self._bufs.get(key)
            if buf is None or buf.numel() < nbytes:
                buf = torch.zeros(max(nbytes, 4096), dtype=torch.uint8, device=device)
                self._bufs[key] = buf
            return buf


_WS = _WorkspacePool()


def _keys_as_i32(rng_keys: torch.Tensor, batch: int) -> torch.Tensor:
    if rng_keys.ndim != 2 or rng_keys.shape[0] != batch or rng_keys.shape[1] != 2:
        raise ValueError(f"rng_keys must be [B, 2] (got {tuple(rng_keys.shape)})")
    if rng_keys.dtype == torch.int32:
        return rng_keys.contiguous()
    if rng_keys.dtype == torch.uint32:
        return rng_keys.contiguous().view(torch.int32)
    if rng_keys.dtype == torch.int64:
        k = rng_keys & 0xFFFFFFFF
        return torch.where(k >= 2**31, k - 2**32, k).to(torch.int32).contiguous()
    raise ValueError(f"rng_keys dtype must be int32/uint32/int64 (got {rng_keys.dtype})")


def _weight_operand(output_weight: torch.Tensor, weight_layout: str | None, hidden_dim: int):
    """Return (tensor, layout code, vocab) for the weight.

    ``weight_layout`` None follows the reference operand ``[H, V]``
    (model.py:759): a transposed view of a contiguous ``[V, H]`` table --
    ``embed_tokens.T`` -- is used in place, zero-copy, on the matrix-core path;
    a contiguous ``[H, V]`` tensor uses the [H, V] layout."""
    if output_weight.ndim != 2:
        raise ValueError("LM-head top1 requires output weight shape [H, V]")
    if weight_layout is None:
        if output_weight.shape[0] != hidden_dim:
            raise ValueError("hidden dimension must match output weight rows")
        vocab = int(output_weight.shape[1])
        if output_weight.stride() == (1, hidden_dim):
            return output_weight.T, _lib.W_VH, vocab
        return output_weight.contiguous(), _lib.W_HV, vocab
    if weight_layout == "vh":
        if output_weight.shape[1] != hidden_dim:
            raise ValueError("hidden dimension must match output weight columns ([V, H] layout)")
        return output_weight.contiguous(), _lib.W_VH, int(output_weight.shape[0])
    if weight_layout == "hv":
        if output_weight.shape[0] != hidden_dim:
            raise ValueError("hidden dimension must match output weight rows")
        return output_weight.contiguous(), _lib.W_HV, int(output_weight.shape[1])
    raise ValueError(f"weight_layout must be None, 'hv' or 'vh' (got {weight_layout!r})")


def reference_reduce_cast(hidden_dtype: torch.dtype, weight_dtype: torch.dtype) -> int:
    """REDUCE_CAST rule of lm_head_triton.py:146-150 (and the bf16 output of jnp.dot)."""
    if hidden_dtype == torch.bfloat16 and weight_dtype == torch.bfloat16:
        return 1
    if hidden_dtype == torch.float16 and weight_dtype == torch.float16:
        return 2
    return 0


def _flatten_hidden(hidden_norm: torch.Tensor, require_3d: bool) -> torch.Tensor:
    if hidden_norm.ndim == 3:
        if int(hidden_norm.shape[1]) != 1:
            raise ValueError("LM-head top1 requires hidden shape [B, 1, H]")
        return hidden_norm.reshape(hidden_norm.shape[0], hidden_norm.shape[2])
    if hidden_norm.ndim == 2 and not require_3d:
        return hidden_norm
    raise ValueError("LM-head top1 requires hidden shape [B, 1, H]")


def _prenorm_operands(norm_weight, act_dtype, hidden_dim: int, dev):
    """The final-RMSNorm prologue's weight (on ``dev``, contiguous) and codes."""
    if norm_weight.ndim != 1 or int(norm_weight.shape[0]) != hidden_dim:
        raise ValueError("norm_weight must be [H]")
    nw = norm_weight.to(dev).contiguous()
    return nw, _dtype_code(nw, "norm_weight"), _TORCH_DTYPES.get(act_dtype)


def lm_head_greedy_top1_hip(hidden_norm: torch.Tensor, output_weight: torch.Tensor, *,
                            weight_layout: str | None = None, reduce_cast: int | None = None,
                            return_best: bool = False, norm_weight: torch.Tensor | None = None,
                            rms_norm_eps: float = 1e-6, act_dtype: torch.dtype = torch.float32):
    """Greedy token ids for ``[B, 1, H] x [H, V]`` without materialising logits.

    Returns int32 ``[B, 1]`` (and the winning logits ``f32[B]`` with
    ``return_best``).  With ``norm_weight`` the input is the pre-norm hidden
    (``hidden_is_normed=False``, model.py:734-762): the library applies the
    final RMSNorm ``rms_norm(x, norm_weight, rms_norm_eps)`` (layers.py:11-29),
    casts to ``act_dtype`` (``lm_head_decode_act_dtype``) and multiplies, in
    one launch on the streaming and bf16 tile paths."""
    x = _flatten_hidden(hidden_norm, require_3d=False)
    batch, hidden_dim = int(x.shape[0]), int(x.shape[1])
    if batch <= 0 or hidden_dim <= 0 or output_weight.numel() == 0:
        raise ValueError("LM-head top1 requires non-empty dimensions")
    hd = _dtype_code(x, "hidden")
    wd = _dtype_code(output_weight, "weight")
    w, layout, vocab = _weight_operand(output_weight, weight_layout, hidden_dim)
    dev = _require_cuda(x, w)
    x = x.contiguous()
    act = x.dtype if norm_weight is None else act_dtype
    if act not in _TORCH_DTYPES:
        raise ValueError(f"unsupported act dtype: {act}")
    rc = reference_reduce_cast(act, w.dtype) if reduce_cast is None else int(reduce_cast)
    out = torch.empty((batch,), dtype=torch.int32, device=dev)
    best = torch.empty((batch,), dtype=torch.float32, device=dev) if return_best else None
    stream = _stream_handle(dev)
    lib = _lib.load()
    best_ptr = best.data_ptr() if best is not None else None
    if norm_weight is None:
        ws = _WS.get(dev, stream, "lm_head", lib.nvjsel_lm_head_workspace_size(batch))
        _lib.call("nvjsel_lm_head_top1", x.data_ptr(), hd, w.data_ptr(), wd, layout, batch, hidden_dim,
                  vocab, rc, out.data_ptr(), best_ptr, ws.data_ptr(), ws.numel(), stream)
    else:
        nw, nd, ad = _prenorm_operands(norm_weight, act, hidden_dim, dev)
        ws = _WS.get(dev, stream, "lm_head", lib.nvjsel_lm_head_prenorm_workspace_size(batch, hidden_dim))
        _lib.call("nvjsel_lm_head_top1_prenorm", x.data_ptr(), hd, nw.data_ptr(), nd, float(rms_norm_eps), ad,
                  w.data_ptr(), wd, layout, batch, hidden_dim, vocab, rc, out.data_ptr(), best_ptr,
                  ws.data_ptr(), ws.numel(), stream)
    ids = out[:, None]
    return (ids, best) if return_best else ids


def _row_stride(logits: torch.Tensor) -> int:
    """Elements between rows of a [B, V] tensor with unit column stride.  A
    size-1 batch dimension may carry any stride (torch keeps numpy's 0 there);
    the library only needs it for B > 1."""
    return int(logits.stride(0)) if int(logits.shape[0]) > 1 else int(logits.shape[1])


def sample_token_ids(logits: torch.Tensor, temperatures: torch.Tensor, rng_keys: torch.Tensor, *,
                     top_k: torch.Tensor | None = None, top_p: torch.Tensor | None = None,
                     noise: torch.Tensor | None = None) -> torch.Tensor:
    """Per-row temperature / top-k / top-p sampling over ``logits [B, V]``
    (or ``[B, 1, V]``).  Returns int32 ``[B]``."""
    if logits.ndim == 3:
        if int(logits.shape[1]) != 1:
            raise ValueError("sampler takes logits [B, V] or [B, 1, V]")
        logits = logits[:, 0, :]
    if logits.ndim != 2:
        raise ValueError("sampler takes logits [B, V] or [B, 1, V]")
    batch, vocab = int(logits.shape[0]), int(logits.shape[1])
    if batch <= 0 or vocab <= 0:
        raise ValueError("sampler requires non-empty dimensions")
    dt = _dtype_code(logits, "logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    dev = _require_cuda(logits, temperatures, rng_keys)
    temps = temperatures.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if temps.numel() != batch:
        raise ValueError("temperatures must have one value per row")
    keys = _keys_as_i32(rng_keys.to(dev), batch)
    tk = None
    if top_k is not None:
        tk = top_k.to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
        if tk.numel() != batch:
            raise ValueError("top_k must have one value per row")
    tp = None
    if top_p is not None:
        tp = top_p.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if tp.numel() != batch:
            raise ValueError("top_p must have one value per row")
    nz = None
    if noise is not None:
        nz = noise.to(device=dev, dtype=torch.float32).contiguous()
        if tuple(nz.shape) != (batch, vocab):
            raise ValueError("noise must be [B, V]")
    out = torch.empty((batch,), dtype=torch.int32, device=dev)
    stream = _stream_handle(dev)
    lib = _lib.load()
    ws = _WS.get(dev, stream, "sample", lib.nvjsel_sample_workspace_size(batch, vocab))
    _lib.call("nvjsel_sample", logits.data_ptr(), dt, batch, vocab, _row_stride(logits),
              temps.data_ptr(), tk.data_ptr() if tk is not None else None,
              tp.data_ptr() if tp is not None else None, keys.data_ptr(),
              nz.data_ptr() if nz is not None else None, out.data_ptr(), ws.data_ptr(), ws.numel(),
              stream)
    return out


def lm_head_sample_token_ids(hidden_norm: torch.Tensor, output_weight: torch.Tensor, *,
                             temperatures: torch.Tensor, rng_keys: torch.Tensor,
                             top_k: torch.Tensor | None = None, top_p: torch.Tensor | None = None,
                             weight_layout: str | None = None,
                             reduce_cast: int | None = None, norm_weight: torch.Tensor | None = None,
                             rms_norm_eps: float = 1e-6,
                             act_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Sample token ids from the LM head (model.py:901-938).

    Without top-k/top-p the projection and the Gumbel-max are fused and no
    logits are written.  With them, the logits are formed once by the
    library's LM-head kernels (rounded as the reference's dot) and handed to
    the sampler.
    ``norm_weight`` selects the pre-norm input as in lm_head_greedy_top1_hip."""
    x = _flatten_hidden(hidden_norm, require_3d=False)
    batch, hidden_dim = int(x.shape[0]), int(x.shape[1])
    if batch <= 0 or hidden_dim <= 0:
        raise ValueError("LM-head sampling requires non-empty dimensions")
    hd = _dtype_code(x, "hidden")
    wd = _dtype_code(output_weight, "weight")
    w, layout, vocab = _weight_operand(output_weight, weight_layout, hidden_dim)
    dev = _require_cuda(x, w)
    x = x.contiguous()
    act = x.dtype if norm_weight is None else act_dtype
    if act not in _TORCH_DTYPES:
        raise ValueError(f"unsupported act dtype: {act}")
    rc = reference_reduce_cast(act, w.dtype) if reduce_cast is None else int(reduce_cast)
    if norm_weight is not None and (top_k is not None or top_p is not None):
        x = rms_norm_hip(x, norm_weight, rms_norm_eps, act)
        norm_weight = None
    if top_k is not None or top_p is not None:
        logits = _dense_logits(x, w, layout, vocab, rc)
        return sample_token_ids(logits, temperatures, rng_keys, top_k=top_k, top_p=top_p)
    temps = temperatures.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if temps.numel() != batch:
        raise ValueError("temperatures must have one value per row")
    keys = _keys_as_i32(rng_keys.to(dev), batch)
    out = torch.empty((batch,), dtype=torch.int32, device=dev)
    stream = _stream_handle(dev)
    lib = _lib.load()
    if norm_weight is None:
        ws = _WS.get(dev, stream, "lm_head", lib.nvjsel_lm_head_workspace_size(batch))
        _lib.call("nvjsel_lm_head_sample", x.data_ptr(), hd, w.data_ptr(), wd, layout, batch, hidden_dim,
                  vocab, rc, temps.data_ptr(), keys.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                  stream)
    else:
        nw, nd, ad = _prenorm_operands(norm_weight, act, hidden_dim, dev)
        ws = _WS.get(dev, stream, "lm_head", lib.nvjsel_lm_head_prenorm_workspace_size(batch, hidden_dim))
        _lib.call("nvjsel_lm_head_sample_prenorm", x.data_ptr(), hd, nw.data_ptr(), nd, float(rms_norm_eps), ad,
                  w.data_ptr(), wd, layout, batch, hidden_dim, vocab, rc, temps.data_ptr(), keys.data_ptr(),
                  out.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    return out


def _dense_logits(x: torch.Tensor, w: torch.Tensor, layout: int, vocab: int, rc: int) -> torch.Tensor:
    """Logits ``[B, V]`` of ``x [B, H]`` against the weight operand, from the
    library's LM-head kernels (nvjsel_lm_head_logits): fp32 accumulation
    rounded as the reference's dot (``rc``); stored bf16 / f16 when they are
    bf16- / f16-rounded (the dtype jnp.dot returns), f32 otherwise."""
    batch, hidden_dim = int(x.shape[0]), int(x.shape[1])
    dev = _require_cuda(x, w)
    x = x.contiguous()
    out_dtype = {1: torch.bfloat16, 2: torch.float16}.get(rc, torch.float32)
    out = torch.empty((batch, vocab), dtype=out_dtype, device=dev)
    _lib.call("nvjsel_lm_head_logits", x.data_ptr(), _dtype_code(x, "hidden"), w.data_ptr(),
              _dtype_code(w, "weight"), layout, batch, hidden_dim, vocab, rc, out.data_ptr(),
              _TORCH_DTYPES[out_dtype], vocab, _stream_handle(dev))
    return out


def lm_head_logits_hip(hidden_norm: torch.Tensor, output_weight: torch.Tensor, *,
                       weight_layout: str | None = None, reduce_cast: int | None = None) -> torch.Tensor:
    """Dense LM-head logits ``[B, V]`` (``jnp.dot(hidden_norm, W)``,
    model.py:765-780): fp32 accumulation; bf16 x bf16 gives bf16 logits and f16 x f16 f16 logits (the
    reference's dot output), other operand types f32 logits."""
    x = _flatten_hidden(hidden_norm, require_3d=False)
    batch, hidden_dim = int(x.shape[0]), int(x.shape[1])
    if batch <= 0 or hidden_dim <= 0 or output_weight.numel() == 0:
        raise ValueError("LM-head logits require non-empty dimensions")
    _dtype_code(x, "hidden")
    _dtype_code(output_weight, "weight")
    w, layout, vocab = _weight_operand(output_weight, weight_layout, hidden_dim)
    rc = reference_reduce_cast(x.dtype, w.dtype) if reduce_cast is None else int(reduce_cast)
    return _dense_logits(x, w, layout, vocab, rc)


def rms_norm_hip(hidden: torch.Tensor, norm_weight: torch.Tensor, eps: float = 1e-6,
                 act_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """The LM-head input of the pre-norm route as a tensor ``[B, H]`` of
    ``act_dtype`` (rms_norm, layers.py:11-29, then the activation cast,
    model.py:758-760), for callers that need dense logits."""
    x = _flatten_hidden(hidden, require_3d=False)
    batch, hidden_dim = int(x.shape[0]), int(x.shape[1])
    if batch <= 0 or hidden_dim <= 0:
        raise ValueError("rms_norm requires non-empty dimensions")
    hd = _dtype_code(x, "hidden")
    dev = _require_cuda(x)
    x = x.contiguous()
    nw, nd, ad = _prenorm_operands(norm_weight, act_dtype, hidden_dim, dev)
    if ad is None:
        raise ValueError(f"unsupported act dtype: {act_dtype}")
    out = torch.empty((batch, hidden_dim), dtype=act_dtype, device=dev)
    _lib.call("nvjsel_rms_norm", x.data_ptr(), hd, nw.data_ptr(), nd, float(eps), ad, batch, hidden_dim,
              out.data_ptr(), _stream_handle(dev))
    return out


def derive_rng_keys(slots: torch.Tensor, counters: torch.Tensor):
    """keys[b] = fold_in(fold_in(PRNGKey(0), slot_b), counter_b) on device.

    Returns (keys int32[B, 2] holding the uint32 bit patterns, counters + 1)."""
    dev = _require_cuda(slots, counters)
    s = slots.to(dtype=torch.int32).reshape(-1).contiguous()
    c = counters.to(dtype=torch.int32).reshape(-1).contiguous()
    if s.numel() != c.numel() or s.numel() == 0:
        raise ValueError("slots and counters must be non-empty and of equal length")
    keys = torch.empty((s.numel(), 2), dtype=torch.int32, device=dev)
    nxt = torch.empty_like(c)
    _lib.call("nvjsel_derive_keys", s.data_ptr(), c.data_ptr(), s.numel(), keys.data_ptr(),
              nxt.data_ptr(), _stream_handle(dev))
    return keys, nxt


def topk_hip(logits: torch.Tensor, k: int):
    """``jax.lax.top_k(logits.astype(float32), k)`` over the last axis of
    ``logits [B, V]`` (or ``[B, 1, V]``): values f32 ``[B, k]`` (the logits'
    own values) and indices int32 ``[B, k]``, by value descending then index
    ascending (NaN first, -0.0 == +0.0)."""
    squeeze = logits.ndim == 3
    if squeeze:
        if int(logits.shape[1]) != 1:
            raise ValueError("topk takes logits [B, V] or [B, 1, V]")
        logits = logits[:, 0, :]
    if logits.ndim != 2:
        raise ValueError("topk takes logits [B, V] or [B, 1, V]")
    batch, vocab = int(logits.shape[0]), int(logits.shape[1])
    k = int(k)
    if batch <= 0 or vocab <= 0:
        raise ValueError("topk requires non-empty dimensions")
    if not 1 <= k <= vocab:
        raise ValueError("top_k must be in [1, vocab]")
    dt = _dtype_code(logits, "logits")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    dev = _require_cuda(logits)
    values = torch.empty((batch, k), dtype=torch.float32, device=dev)
    indices = torch.empty((batch, k), dtype=torch.int32, device=dev)
    stream = _stream_handle(dev)
    lib = _lib.load()
    ws = _WS.get(dev, stream, "sample", lib.nvjsel_topk_workspace_size(batch, vocab))
    _lib.call("nvjsel_topk", logits.data_ptr(), dt, batch, vocab, _row_stride(logits), k, values.data_ptr(),
              indices.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    if squeeze:
        return values[:, None, :], indices[:, None, :]
    return values, indices


def lm_head_token_ids_and_topk(hidden: torch.Tensor, output_weight: torch.Tensor, *, top_k: int = 0,
                               norm_weight: torch.Tensor | None = None, rms_norm_eps: float = 1e-6,
                               act_dtype: torch.dtype = torch.float32, weight_layout: str | None = None,
                               reduce_cast: int | None = None):
    """Greedy token ids and optional top-k of the LM head (model.py:833-898).

    ``hidden [B, W, H]`` (W > 1: MTP / verifier width, flattened to B*W rows as
    model.py:862-865) or ``[B, H]``; ``norm_weight`` given: pre-norm input.
    ``top_k == 0``: the fused greedy route, returns ``(ids int32[B, W], None,
    None)``.  ``top_k > 0``: dense logits (the reference's dot: bf16 x bf16
    rounds to bf16) and ``topk_hip``; returns ``(ids, values f32[B, W, k],
    indices int32[B, W, k])`` with ``ids = indices[..., 0]``, the argmax."""
    if hidden.ndim == 2:
        hidden = hidden[:, None, :]
    if hidden.ndim != 3:
        raise ValueError("hidden must be [B, W, H] or [B, H]")
    batch, width, hidden_dim = (int(d) for d in hidden.shape)
    flat = hidden.reshape(batch * width, hidden_dim)
    if int(top_k) == 0:
        ids = lm_head_greedy_top1_hip(flat, output_weight, weight_layout=weight_layout, reduce_cast=reduce_cast,
                                      norm_weight=norm_weight, rms_norm_eps=rms_norm_eps, act_dtype=act_dtype)
        return ids.reshape(batch, width), None, None
    w, layout, vocab = _weight_operand(output_weight, weight_layout, hidden_dim)
    x = flat if norm_weight is None else rms_norm_hip(flat, norm_weight, rms_norm_eps, act_dtype)
    rc = reference_reduce_cast(x.dtype, w.dtype) if reduce_cast is None else int(reduce_cast)
    logits = _dense_logits(x.contiguous(), w, layout, vocab, rc)
    values, indices = topk_hip(logits, int(top_k))
    ids = indices[:, 0].reshape(batch, width)
    return ids, values.reshape(batch, width, -1), indices.reshape(batch, width, -1)


def mtp_greedy_top1_token_ids(x_normed: torch.Tensor, output_weight: torch.Tensor, *,
                              weight_layout: str | None = None) -> torch.Tensor:
    """MTP draft seeding with the HIP top-1 (_mtp_greedy_top1_token_ids,
    mtp/mtp_layer.py:220-248, its Triton branch): ``x_normed [B, T, H]`` is
    cast to the weight's dtype (the contract of
    tests/test_mtp_layer_contract.py:155-178), T > 1 is flattened to B*T rows
    and reshaped back.  Returns int32 ``[B, T]``."""
    if x_normed.ndim != 3:
        raise ValueError("HIP MTP greedy top1 expects hidden shape [B, T, H]")
    batch, seq_len, hidden_dim = (int(d) for d in x_normed.shape)
    flat = x_normed.reshape(batch * seq_len, 1, hidden_dim).to(output_weight.dtype)
    ids = lm_head_greedy_top1_hip(flat, output_weight, weight_layout=weight_layout)
    return ids.reshape(batch, seq_len)


DERIVE_KEYS_TABLE_MAX_BATCH = 8192  # nvjsel_derive_keys_table's limit (include/nvjsel.h)


def derive_rng_keys_from_table(slots: torch.Tensor, counter_table: torch.Tensor) -> torch.Tensor:
    """Keys for the rows' slots from the device-resident counter table, which
    is advanced in place (model_executor.py:3593-3619).  ``counter_table`` is
    int32 ``[num_slots]`` on the device; returns keys int32 ``[B, 2]`` (uint32
    bit patterns) for the samplers' ``rng_keys``."""
    dev = _require_cuda(slots, counter_table)
    if counter_table.dtype != torch.int32 or counter_table.ndim != 1 or not counter_table.is_contiguous():
        raise ValueError("counter_table must be a contiguous int32 [num_slots] tensor")
    s = slots.to(dtype=torch.int32).reshape(-1).contiguous()
    if s.numel() == 0 or counter_table.numel() == 0:
        raise ValueError("slots and counter_table must be non-empty")
    if s.numel() > DERIVE_KEYS_TABLE_MAX_BATCH:
        # one launch gathers every counter before any is written (LDS staging)
        raise ValueError(f"derive_rng_keys_from_table serves at most {DERIVE_KEYS_TABLE_MAX_BATCH} rows per call")
    keys = torch.empty((s.numel(), 2), dtype=torch.int32, device=dev)
    _lib.call("nvjsel_derive_keys_table", s.data_ptr(), s.numel(), counter_table.data_ptr(),
              counter_table.numel(), keys.data_ptr(), _stream_handle(dev))
    return keys


def reset_rng_counters(counter_table: torch.Tensor, slots) -> None:
    """Zero the counters of released / reused slots
    (_flush_resident_rng_counter_resets, model_runner.py:4801-4815)."""
    idx = torch.as_tensor(list(slots) if not torch.is_tensor(slots) else slots, dtype=torch.long,
                          device=counter_table.device).reshape(-1)
    idx = idx[idx >= 0]
    if idx.numel():
        counter_table.index_fill_(0, idx, 0)
