"""MI355X (gfx950) FlashAttention-2 forward — Python entry point.

Drop-in for the reference package ``flash_attention_runtime``
(python/flash_attention_runtime/__init__.py:30-38): ``forward(q, k, v, o=None)``
returns ``o`` and ``forward_timed(q, k, v, o=None)`` returns ``(o, ms)``, with
q, k, v laid out [B, H, N, D] on the GPU.  Keyword-only extensions:
``causal`` (top-left aligned mask), ``softmax_scale`` (default 1/sqrt(D), as
the reference), ``return_lse`` (also return the natural-log logsumexp,
fp32 [B, H, N]) and ``split_kv`` (default True: problems whose grid would
leave most CUs idle behind a few long q-tiles split their key ranges across
workgroups, with an fp32 workspace from torch's allocator; False always runs
one workgroup per q-tile).

The reference JIT-compiles its CUDA extension on first use
(``__init__.py:10-27``); here the HIP library ``libfa_mi355x.so`` and the
torch binding ``_C`` are prebuilt in this directory by ``build.py``.  There is
no fallback: if the native extension is missing, importing this package
raises, so a GPU run can never silently fall back to a non-HIP path.
"""
from __future__ import annotations

import glob
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))


def _load_ext():
    candidates = glob.glob(os.path.join(_HERE, "_C*.so"))
    if not candidates:
        raise ImportError(
            "flash_attention_runtime: native extension _C is not built in "
            f"{_HERE}; run `python __graft_entry__.py build` (or "
            "`python flash-attention_amd/build.py`) first"
        )
    from . import _C  # noqa: WPS433  (the prebuilt torch extension)

    return _C


_EXT = _load_ext()


def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor | None = None,
    *,
    causal: bool = False,
    softmax_scale: float | None = None,
    return_lse: bool = False,
    split_kv: bool = True,
):
    """softmax(q k^T * scale [+ causal mask]) v.

    Returns ``o`` (same dtype as q), or ``(o, lse)`` when ``return_lse``.
    """
    res = _EXT.forward(q, k, v, o, False, causal=causal, softmax_scale=softmax_scale,
                       return_lse=return_lse, split_kv=split_kv)
    return (res[0], res[2]) if return_lse else res[0]


def forward_timed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    o: torch.Tensor | None = None,
    *,
    causal: bool = False,
    softmax_scale: float | None = None,
    return_lse: bool = False,
    split_kv: bool = True,
):
    """Like ``forward`` but also returns the kernel time in ms measured with
    two HIP events on the current stream (blocks until the kernel ends).

    Returns ``(o, ms)``, or ``(o, ms, lse)`` when ``return_lse``.
    """
    return tuple(_EXT.forward(q, k, v, o, True, causal=causal, softmax_scale=softmax_scale,
                              return_lse=return_lse, split_kv=split_kv))


def device_info(device: int = 0) -> dict:
    """hipDeviceProp summary plus the derived dense fp16/bf16 MFMA peak
    (replaces the reference's utils/get_gpu_hardware_param.cu)."""
    return dict(_EXT.device_info(device))


def version() -> str:
    return _EXT.version()


__all__ = ["forward", "forward_timed", "device_info", "version"]
