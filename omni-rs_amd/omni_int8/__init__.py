"""MI355X (gfx950) int8 quantised matmul — host-side mirror of omni-rs's operator API.

The functions here keep the reference operator's names, argument meaning and
``None`` convention and hand device tensors to libomni_int8.so through its C
ABI. Every op runs the hand-written HIP kernels; nothing falls back to a CPU
path: a missing library, a non-gfx950 device or a CPU tensor raises.

Reference interface (GoooIce/omni-rs):
  try_int8_gemm            crates/omni-kernel/src/int8_matmul.rs:505-560
  Int8Linear / hadamard    crates/qwen-image/src/convrot.rs:70-160 (see convrot.py)
  fp16 try_linear (x2)     crates/breeze-tts/src/metal_depth.rs:84-123,
                           crates/qwen-image/src/metal_tensorops.rs:161-203 (see f16.py)
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import (OMNI_F16, OMNI_F32, OMNI_LOWERING_AUTO, OMNI_LOWERING_MFMA,
                   OMNI_LOWERING_SCALAR, OMNI_NOT_HANDLED, OMNI_OK, OmniError)

__all__ = [
    "try_int8_gemm", "quantize_rows", "w8a8_gemm", "w8a16_linear", "w4a16_linear", "pack_i8",
    "arch_supported", "lowering", "OmniError",
    "OMNI_LOWERING_AUTO", "OMNI_LOWERING_MFMA", "OMNI_LOWERING_SCALAR",
]


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: Optional[torch.Tensor]) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise OmniError(_lib.OMNI_BAD_ARGUMENT, "tensors must live on the GPU")
        if device is None:
            device = t.device
        elif t.device != device:
            # crates/omni-kernel/src/lib.rs:83-88 asserts one device for all inputs
            raise OmniError(_lib.OMNI_BAD_ARGUMENT, "tensors live on different devices")
    if device is None:
        raise OmniError(_lib.OMNI_BAD_ARGUMENT, "no tensor given")
    return device


def arch_supported(device: int = 0) -> bool:
    """gfx950 probe, cached per device (int8_tensorops.rs:26-43 analog)."""
    return bool(_lib.lib().omni_int8_arch_supported(device))


def lowering(width: int) -> int:
    """W8A8 lowering the library picks for this width (int8_tensorops.rs:15-20 analog)."""
    return _lib.lib().omni_w8a8_lowering(width)


def pack_i8(codes: torch.Tensor) -> torch.Tensor:
    """Four int8 codes per int32 word, first code in the lowest byte
    (crates/qwen-image/src/convrot.rs:151-160). Byte-identical to the codes, so
    this is a reinterpretation, not a copy."""
    if codes.dtype != torch.int8 or codes.numel() % 4:
        raise ValueError("pack_i8 wants int8 codes, a multiple of 4 of them")
    return codes.contiguous().view(torch.int32).reshape(-1)


def quantize_rows(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Per-row symmetric int8 quantisation (int8_matmul.rs:23-118).

    x: [rows, width] f32 or f16 on the GPU -> (codes int8 [rows, width],
    row_scale f32 [rows], row_sum int32 [rows])."""
    if x.dim() != 2:
        raise ValueError("x must be 2-D")
    device = _require_gpu(x)
    if x.stride(1) != 1:
        x = x.contiguous()
    rows, width = x.shape
    dtype = {torch.float32: OMNI_F32, torch.float16: OMNI_F16}.get(x.dtype)
    if dtype is None:
        x = x.float()
        dtype = OMNI_F32
    words = torch.empty((rows, width // 4), dtype=torch.int32, device=device)
    scale = torch.empty(rows, dtype=torch.float32, device=device)
    total = torch.empty(rows, dtype=torch.int32, device=device)
    st = _lib.check(_lib.lib().omni_int8_quantize_rows(
        _ptr(x), dtype, rows, width, x.stride(0), _ptr(words), _ptr(scale), _ptr(total),
        _stream(device)))
    if st == OMNI_NOT_HANDLED:
        raise ValueError(_lib.last_error())
    return words.view(torch.int8).reshape(rows, width), scale, total


def _vector(t: Optional[torch.Tensor], n: int, dtype: torch.dtype, name: str) -> Optional[torch.Tensor]:
    """A 1-D operand of n elements of `dtype`, contiguous (a copy if strided).
    The caller keeps the returned tensor alive until the library call that
    reads it has returned."""
    if t is None:
        return None
    if t.numel() != n or t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype} [{n}], got {t.dtype} {list(t.shape)}")
    return t.reshape(-1).contiguous()


def w8a8_gemm(codes: torch.Tensor, row_scale: torch.Tensor, row_sum: Optional[torch.Tensor],
              w: torch.Tensor, w_scale: torch.Tensor, w_zero: Optional[torch.Tensor] = None,
              bias: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.float32,
              acc_dump: bool = False, lowering: int = OMNI_LOWERING_AUTO):
    """int8 x int8 -> int32 GEMM with the fused reference epilogue
    (int8_matmul.rs:145-373). codes int8 [rows, width]; w int8 [columns, width]
    (or its packed int32 words); row_scale f32 [rows]; row_sum int32 [rows]
    (may be None when w_zero is None); w_scale f32 [columns]; w_zero int32
    [columns]; bias f32 [columns]. Returns out (and the int32 accumulators if
    acc_dump)."""
    device = _require_gpu(codes, row_scale, row_sum, w, w_scale, w_zero, bias)
    if codes.dim() != 2 or codes.dtype != torch.int8:
        raise ValueError("codes must be int8 [rows, width]")
    rows, width = codes.shape
    if w.dtype == torch.int32:
        w = w.view(torch.int8)
    if w.dtype != torch.int8:
        raise ValueError("w must be int8 [columns, width] or its int32 words")
    w = w.reshape(-1, width) if w.numel() else w.reshape(0, width)
    columns = w.shape[0]
    # Every operand the library reads is bound to a local here, so that a
    # contiguous copy stays allocated until the call has returned (the launch
    # is stream-ordered; the caching allocator may not hand the block out
    # again before then).
    codes_c = codes.contiguous()
    w_c = w.contiguous()
    row_scale_c = _vector(row_scale, rows, torch.float32, "row_scale")
    row_sum_c = _vector(row_sum, rows, torch.int32, "row_sum")
    w_scale_c = _vector(w_scale, columns, torch.float32, "w_scale")
    w_zero_c = _vector(w_zero, columns, torch.int32, "w_zero")
    bias_c = _vector(bias, columns, torch.float32, "bias")
    if w_zero_c is not None and row_sum_c is None:
        raise ValueError("row_sum is required when w_zero is given")
    odt = {torch.float32: OMNI_F32, torch.float16: OMNI_F16}[out_dtype]
    out = torch.empty((rows, columns), dtype=out_dtype, device=device)
    acc = torch.empty((rows, columns), dtype=torch.int32, device=device) if acc_dump else None
    L = _lib.lib()
    ws_bytes = L.omni_w8a8_gemm_workspace_size(rows, columns, width) if lowering != OMNI_LOWERING_SCALAR else 0
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    st = _lib.check(L.omni_w8a8_gemm_ws(
        _ptr(codes_c), _ptr(row_scale_c), _ptr(row_sum_c), _ptr(w_c), _ptr(w_scale_c),
        _ptr(w_zero_c), _ptr(bias_c), rows, columns, width, _ptr(out), odt, _ptr(acc),
        lowering, _ptr(workspace), ws_bytes, _stream(device)))
    if st == OMNI_NOT_HANDLED:
        raise ValueError(_lib.last_error())
    return (out, acc) if acc_dump else out


def try_int8_gemm(x: torch.Tensor, w_packed: torch.Tensor, w_scale: torch.Tensor,
                  w_zero: torch.Tensor) -> Optional[torch.Tensor]:
    """``x @ W^T`` after per-row symmetric int8 quantisation of ``x``.

    Mirrors ``omni_kernel::int8_matmul::try_int8_gemm``
    (crates/omni-kernel/src/int8_matmul.rs:505-560): ``w_packed`` holds
    ``n * (k / 4)`` little-endian int8 groups; ``w_scale`` and ``w_zero`` are
    per output row. Returns an f32 ``[rows, n]`` tensor, or ``None`` when the
    shapes disagree (:517-521). Float inputs of any dtype are cast to f32
    (:525-526; f16 is passed through, since it is exact in f32); integer
    inputs may be int32 or int64 (int64 is truncated to int32 as read_i32,
    :587-595, does)."""
    rows, width = x.shape
    columns = w_scale.shape[0]
    if width % 4 != 0 or w_packed.shape[0] != columns * width // 4 or w_zero.shape[0] != columns:
        return None
    device = _require_gpu(x, w_packed, w_scale, w_zero)
    if x.dtype not in (torch.float32, torch.float16):
        x = x.float()
    x = x.contiguous()
    w_packed = w_packed.to(torch.int32).contiguous()
    w_scale = w_scale.to(torch.float32).contiguous()
    w_zero = w_zero.to(torch.int32).contiguous()
    L = _lib.lib()
    # With room for the split-K partial sums the GEMM splits K where that
    # pays.
    ws_bytes = L.omni_try_int8_gemm_split_workspace_size(rows, columns, width)
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    out = torch.empty((rows, columns), dtype=torch.float32, device=device)
    st = _lib.check(L.omni_try_int8_gemm(
        _ptr(x), OMNI_F16 if x.dtype == torch.float16 else OMNI_F32, rows, width,
        _ptr(w_packed), w_packed.shape[0], _ptr(w_scale), columns, _ptr(w_zero), columns,
        _ptr(out), _ptr(workspace), ws_bytes, _stream(device)))
    if st == OMNI_NOT_HANDLED:
        return None
    return out


def w8a16_linear(x: torch.Tensor, w: torch.Tensor, scale: torch.Tensor,
                 bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Weight-only int8 linear: f16(scale[n] * sum_k x[m,k] * w[n,k] + bias[n]).

    x f16 [rows, width] (leading dims are flattened), w int8 [columns, width],
    scale/bias f16 [columns] -> f16 [..., columns]. Decode shapes (rows <= 4)
    run the HBM-bound GEMV, larger ones the fp16-MFMA GEMM."""
    lead = x.shape[:-1]
    width = x.shape[-1]
    x2 = x.reshape(-1, width)
    device = _require_gpu(x2, w, scale, bias)
    if x2.dtype != torch.float16 or w.dtype != torch.int8 or scale.dtype != torch.float16:
        raise ValueError("w8a16_linear wants f16 x, int8 w, f16 scale")
    if bias is not None and bias.dtype != torch.float16:
        raise ValueError("bias must be f16")
    columns = w.shape[0]
    if w.shape[1] != width or scale.numel() != columns or (bias is not None and bias.numel() != columns):
        raise ValueError("w8a16_linear: shapes disagree")
    # contiguous copies bound to locals: alive until the call has returned
    x2 = x2.contiguous()
    w = w.contiguous()
    scale_c = scale.reshape(-1).contiguous()
    bias_c = None if bias is None else bias.reshape(-1).contiguous()
    out = torch.empty((x2.shape[0], columns), dtype=torch.float16, device=device)
    L = _lib.lib()
    ws_bytes = L.omni_w8a16_gemm_workspace_size(x2.shape[0], columns, width)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    st = _lib.check(L.omni_w8a16_gemm_ws(
        _ptr(x2), _ptr(w), _ptr(scale_c), _ptr(bias_c), x2.shape[0], columns, width, _ptr(out),
        _ptr(workspace), ws_bytes, _stream(device)))
    if st == OMNI_NOT_HANDLED:
        raise ValueError(_lib.last_error())
    return out.reshape(*lead, columns)


def w4a16_linear(x: torch.Tensor, w_packed: torch.Tensor, scale: torch.Tensor,
                 bias: Optional[torch.Tensor] = None, group: int = 128) -> torch.Tensor:
    """Weight-only int4 linear in the MiniCPM-V pack-quantized format
    (crates/minicpm-v/src/quant.rs:22-201): ``x @ W^T`` with
    ``W[n][k] = q[n][k] * scale[n][k // group]``.

    x f16 [..., width]; w_packed uint8 [columns, width // 2] (two values per
    byte, low nibble first, stored plus 8); scale bf16 [columns, width // group];
    bias f16 [columns] -> f16 [..., columns]."""
    lead = x.shape[:-1]
    width = x.shape[-1]
    x2 = x.reshape(-1, width)
    device = _require_gpu(x2, w_packed, scale, bias)
    if x2.dtype != torch.float16 or w_packed.dtype != torch.uint8 or scale.dtype != torch.bfloat16:
        raise ValueError("w4a16_linear wants f16 x, uint8 packed weights, bf16 scales")
    columns = w_packed.shape[0]
    if (w_packed.shape[-1] * 2 != width or scale.numel() != columns * (width // group)
            or (bias is not None and (bias.dtype != torch.float16 or bias.numel() != columns))):
        raise ValueError("w4a16_linear: shapes disagree")
    # contiguous copies bound to locals: alive until the call has returned
    x2 = x2.contiguous()
    w_c = w_packed.contiguous()
    scale_c = scale.contiguous()
    bias_c = None if bias is None else bias.reshape(-1).contiguous()
    out = torch.empty((x2.shape[0], columns), dtype=torch.float16, device=device)
    L = _lib.lib()
    ws_bytes = L.omni_w4a16_gemm_workspace_size(x2.shape[0], columns, width, group)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device) if ws_bytes else None
    st = _lib.check(L.omni_w4a16_gemm_ws(
        _ptr(x2), _ptr(w_c), _ptr(scale_c), group, _ptr(bias_c), x2.shape[0], columns, width,
        _ptr(out), _ptr(workspace), ws_bytes, _stream(device)))
    if st == OMNI_NOT_HANDLED:
        raise ValueError(_lib.last_error())
    return out.reshape(*lead, columns)
