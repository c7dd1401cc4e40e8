"""nvjsel -- MI355X-native decode-step token selection (LM-head top-1 + sampler).

Import with ``nano-vllm-jax_amd`` on ``sys.path`` (the repo-root entry points
and tests do this).  The compute lives in ``libnvjsel.so`` (HIP, gfx950); see
``include/nvjsel.h`` for the C ABI.
"""
from ._lib import NativeLibraryMissing, NvjselError, load
from .registry import (
    KernelBackendUnavailable,
    available_backends,
    lm_head_greedy_top1_impl,
    mtp_lm_head_greedy_top1_impl,
    select_token_selection_backend,
)
from .selection import (
    derive_rng_keys,
    derive_rng_keys_from_table,
    lm_head_greedy_top1_hip,
    lm_head_logits_hip,
    lm_head_sample_token_ids,
    lm_head_token_ids_and_topk,
    mtp_greedy_top1_token_ids,
    reference_reduce_cast,
    reset_rng_counters,
    rms_norm_hip,
    sample_token_ids,
    topk_hip,
)

__all__ = [
    "NativeLibraryMissing",
    "NvjselError",
    "KernelBackendUnavailable",
    "available_backends",
    "derive_rng_keys",
    "derive_rng_keys_from_table",
    "load",
    "lm_head_greedy_top1_hip",
    "lm_head_greedy_top1_impl",
    "lm_head_logits_hip",
    "lm_head_sample_token_ids",
    "lm_head_token_ids_and_topk",
    "mtp_greedy_top1_token_ids",
    "mtp_lm_head_greedy_top1_impl",
    "reference_reduce_cast",
    "reset_rng_counters",
    "rms_norm_hip",
    "sample_token_ids",
    "select_token_selection_backend",
    "topk_hip",
]
