"""fp16 linears on the W8A16 kernels with f16 weights.

Two entry points, each mirroring one ``try_linear`` of the reference with its
guard and ``None`` convention:

  depth_try_linear      crates/breeze-tts/src/metal_depth.rs:84-123
                        (decode GEMV, 1..=64 rows, K % 32 == 0, N <= 4096)
  tensorops_try_linear  crates/qwen-image/src/metal_tensorops.rs:161-203
                        (DiT GEMM, 256..=65535 rows, K and N in 4096..=12288,
                        multiples of 64; OMNI_QWEN_TENSOROPS=0 turns it off)

``w`` is the ``[k, n]`` weight the reference passes: the transposed view of a
Linear's output-major ``[n, k]`` weight. Such a view is handed to the kernel
as it lies; any other layout is first copied output-major (the reference
sends that case to its stock matmul instead, metal_depth.rs:42-47,
metal_tensorops.rs:128-131). The result is ``f16(x @ w)`` with f32
accumulation. Tensors off the GPU give ``None``, as the reference's device
check does (metal_depth.rs:88-90); a missing library raises.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from ._lib import OMNI_NOT_HANDLED

__all__ = ["depth_try_linear", "tensorops_try_linear"]


def _run(entry: str, x: torch.Tensor, w: torch.Tensor) -> Optional[torch.Tensor]:
    if x.device.type != "cuda" or w.device != x.device:
        return None
    if x.dim() < 1 or w.dim() != 2 or x.dtype != torch.float16 or w.dtype != torch.float16:
        return None
    k, n = w.shape
    if x.shape[-1] != k:
        return None
    lead = x.shape[:-1]
    rows = math.prod(lead)
    x2 = x.reshape(rows, k).contiguous()
    wt = w.t()
    if not wt.is_contiguous():
        wt = wt.contiguous()
    out = torch.empty((rows, n), dtype=torch.float16, device=x.device)
    st = _lib.check(getattr(_lib.lib(), entry)(
        x2.data_ptr(), wt.data_ptr(), rows, n, k, out.data_ptr(),
        torch.cuda.current_stream(x.device).cuda_stream))
    if st == OMNI_NOT_HANDLED:
        return None
    return out.reshape(*lead, n)


def depth_try_linear(x: torch.Tensor, w: torch.Tensor) -> Optional[torch.Tensor]:
    """Breeze depth-decoder GEMV: x f16 [..., k], w f16 [k, n] -> f16 [..., n],
    or None outside 1..=64 rows, k % 32 == 0, 1..=4096 columns."""
    return _run("omni_f16_gemv", x, w)


def tensorops_try_linear(x: torch.Tensor, w: torch.Tensor) -> Optional[torch.Tensor]:
    """Qwen-Image DiT GEMM: x f16 [..., k], w f16 [k, n] -> f16 [..., n], or
    None outside 256..=65535 rows, k and n multiples of 64 in 4096..=12288."""
    return _run("omni_f16_gemm", x, w)
