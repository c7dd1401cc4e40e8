"""Backend selection for token selection.

Mirrors the reference's declarative backend table and its strict-fail
convention (nanovllm_jax/kernels/registry.py:15-110, 182-209) and the
``lm_head_greedy_top1_impl`` value set (nanovllm_jax/model.py:369-380), with a
``"hip"`` entry that is this package.  There is no pure-JAX path in this build,
so an unavailable HIP library always raises ``KernelBackendUnavailable`` --
never a silent fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

from . import _lib


class KernelBackendUnavailable(RuntimeError):
    """Raised when the requested token-selection backend cannot run."""


@dataclass(frozen=True)
class KernelBackendSpec:
    name: str
    aliases: tuple[str, ...]
    required_modules: tuple[str, ...]
    provided_kernels: tuple[str, ...]
    implemented: bool
    description: str


@dataclass(frozen=True)
class KernelBackendStatus:
    """The reference's status record (kernels/registry.py:30-52), field for
    field.  ``missing_modules`` names the native library when it cannot load;
    ``fallback`` is always None: this backend never falls back."""

    requested: str
    selected: str
    available: bool
    implemented: bool
    external_kernels_enabled: bool
    missing_modules: tuple[str, ...] = ()
    provided_kernels: tuple[str, ...] = ()
    fallback: str | None = None
    reason: str = ""

    def as_dict(self) -> dict[str, object]:
        return {
            "requested": self.requested,
            "selected": self.selected,
            "available": self.available,
            "implemented": self.implemented,
            "external_kernels_enabled": self.external_kernels_enabled,
            "missing_modules": list(self.missing_modules),
            "provided_kernels": list(self.provided_kernels),
            "fallback": self.fallback,
            "reason": self.reason,
        }


_SPECS = {
    "hip": KernelBackendSpec(
        name="hip",
        aliases=("hip", "rocm", "nvjsel", "mi355x", "gfx950", "auto"),
        required_modules=(),
        provided_kernels=(
            "lm_head_greedy_top1",
            "lm_head_greedy_top1_prenorm",
            "lm_head_sample",
            "lm_head_topk",
            "mtp_greedy_top1",
            "sample_topk_topp",
            "derive_rng_keys",
            "lm_head_logits",
        ),
        implemented=True,
        description="Hand-written HIP kernels for gfx950 behind the libnvjsel C ABI.",
    ),
}
_ALIASES = {a: n for n, s in _SPECS.items() for a in s.aliases}


def lm_head_greedy_top1_impl(value: str | None) -> str:
    """Normalise an ``lm_head_greedy_top1_impl`` setting (model.py:369-380 plus "hip")."""
    v = str(value or "jax").strip().lower()
    if v in {"", "0", "false", "no", "off", "none", "jax", "reference"}:
        return "jax"
    if v in {"triton", "triton_tensorcore", "triton_epilogue"}:
        return "triton"
    if v in {"cutlass", "cutlass_top1", "cutlass_fused_gemm", "fused_gemm"}:
        return "cutlass"
    if v in {"hip", "hip_mfma", "rocm", "nvjsel"}:
        return "hip"
    raise ValueError(
        "lm_head_greedy_top1_impl must be jax, triton, cutlass, or hip, "
        f"got {value!r}")


def mtp_lm_head_greedy_top1_impl(value: str | None) -> str:
    """Normalise ``mtp_lm_head_greedy_top1_impl`` (mtp/mtp_layer.py:225-247 plus "hip")."""
    v = str(value or "jax").strip().lower()
    if v in {"jax", "", "none"}:
        return "jax"
    if v in {"triton", "triton_tensorcore", "triton_top1"}:
        return "triton"
    if v in {"cutlass", "cutlass_top1", "cutlass_fused_gemm", "fused_gemm"}:
        return "cutlass"
    if v in {"hip", "hip_mfma", "rocm", "nvjsel"}:
        return "hip"
    raise ValueError(f"unsupported MTP greedy top1 implementation: {value!r}")


def _normalize(name: str | None) -> str:
    v = (name or "hip").strip().lower()
    try:
        return _ALIASES[v]
    except KeyError:
        valid = ", ".join(sorted(_ALIASES))
        raise ValueError(f"Unknown token-selection backend {name!r}; expected one of: {valid}") from None


def backend_status(name: str | None = None) -> KernelBackendStatus:
    n = _normalize(name)
    spec = _SPECS[n]
    try:
        _lib.load()
        return KernelBackendStatus(requested=name or n, selected=n, available=True, implemented=spec.implemented,
                                   external_kernels_enabled=True, provided_kernels=spec.provided_kernels,
                                   reason=f"{n} backend selected")
    except Exception as exc:  # library missing or ABI mismatch
        return KernelBackendStatus(requested=name or n, selected=n, available=False, implemented=spec.implemented,
                                   external_kernels_enabled=False, missing_modules=(_lib.LIB_PATH.name,),
                                   provided_kernels=spec.provided_kernels, reason=str(exc))


def select_token_selection_backend(name: str | None = None, *, strict: bool = True) -> KernelBackendStatus:
    """Resolve the backend; raises ``KernelBackendUnavailable`` when it cannot run
    (``strict=False`` returns the unavailable status instead)."""
    st = backend_status(name)
    if strict and not st.available:
        raise KernelBackendUnavailable(st.reason)
    return st


def available_backends() -> dict[str, KernelBackendStatus]:
    return {n: backend_status(n) for n in _SPECS}
