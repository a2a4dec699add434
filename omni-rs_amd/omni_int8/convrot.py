"""INT8-ConvRot linear layers (Qwen-Image-2.1-Turbo DiT) on the gfx950 kernels.

Host-side mirror of ``crates/qwen-image/src/convrot.rs``: the layer keeps the
reference's names and contract (``GROUP``, ``hadamard``, ``Int8Linear`` with
``forward`` = rotate by the group-256 Hadamard, then ``try_int8_gemm``, then
cast to the model precision). On the GPU the rotation is not a matmul: it is
fused into the quantisation pass (``omni_convrot_quantize_rows``) and the
whole layer is one C-ABI call (``omni_convrot_linear``).
"""
from __future__ import annotations

import json
import os
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _lib
from ._lib import OMNI_F16, OMNI_F32, OMNI_NOT_HANDLED

GROUP = 256  # crates/qwen-image/src/convrot.rs:12
FILE_NAME = "Qwen-Image-2.1-Turbo-INT8-ConvRot.safetensors"  # convrot.rs:13


class CheckpointError(ValueError):
    """A malformed checkpoint, a missing tensor or one of the wrong dtype
    (the reference's Error::Checkpoint, src/weights.rs:316-320, 429-462)."""


class ConfigError(ValueError):
    """A layer whose tensors do not fit its declared shape (the reference's
    Error::Config, crates/qwen-image/src/convrot.rs:39-50)."""


# safetensors dtype tag -> numpy dtype (little-endian payloads)
_DTYPES = {"I8": np.int8, "U8": np.uint8, "I16": np.int16, "I32": np.int32, "I64": np.int64,
           "F16": np.float16, "BF16": np.uint16, "F32": np.float32, "F64": np.float64,
           "BOOL": np.bool_}


class SafetensorsFile:
    """Read-only memory map of one safetensors file: an 8-byte little-endian
    header length, a JSON header naming each tensor's dtype, shape and byte
    range, then the payload. Mirrors the raw accessors of src/weights.rs
    (open_file :301-304, raw_i8 :429-442, raw_f32 :444-462): host views of
    one tensor, checked for dtype and length."""

    def __init__(self, path: str):
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        if self._map.size < 8:
            raise CheckpointError(f"{path}: too short for a safetensors header")
        n = int(self._map[:8].view("<u8")[0])
        if n > self._map.size - 8:
            raise CheckpointError(f"{path}: header length {n} exceeds the file")
        try:
            header = json.loads(bytes(self._map[8:8 + n]).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise CheckpointError(f"{path}: bad header: {e}") from None
        self._base = 8 + n
        self.metadata = header.pop("__metadata__", {})
        self._entries: Dict[str, Tuple[str, Tuple[int, ...], int, int]] = {}
        for name, e in header.items():
            try:
                dtype, shape, (begin, end) = e["dtype"], tuple(int(d) for d in e["shape"]), e["data_offsets"]
            except (KeyError, TypeError, ValueError):
                raise CheckpointError(f"{path}: bad header entry for {name}") from None
            if not (0 <= begin <= end <= self._map.size - self._base):
                raise CheckpointError(f"{path}: {name} lies outside the file")
            self._entries[name] = (dtype, shape, int(begin), int(end))

    def names(self):
        return sorted(self._entries)

    def __contains__(self, name: str) -> bool:
        return name in self._entries

    def _view(self, name: str, want: str) -> Tuple[Tuple[int, ...], np.ndarray]:
        if name not in self._entries:
            raise CheckpointError(f"missing tensor {name}")
        dtype, shape, begin, end = self._entries[name]
        if dtype != want:
            raise CheckpointError(f"{name}: expected {want}, got {dtype}")
        np_dtype = np.dtype(_DTYPES[want]).newbyteorder("<")
        count = int(np.prod(shape)) if shape else 1
        if end - begin != count * np_dtype.itemsize:
            raise CheckpointError(f"{name}: payload of {end - begin} bytes for shape {list(shape)}")
        data = self._map[self._base + begin:self._base + end].view(np_dtype)
        return shape, data

    def raw_i8(self, name: str) -> Tuple[Tuple[int, ...], np.ndarray]:
        """(shape, flat int8 view) of one I8 tensor (weights.rs:429-442)."""
        return self._view(name, "I8")

    def raw_f32(self, name: str) -> Tuple[Tuple[int, ...], np.ndarray]:
        """(shape, flat f32 view) of one F32 tensor, any rank (weights.rs:444-462)."""
        return self._view(name, "F32")


class ConvRotFile:
    """The INT8-ConvRot checkpoint of Qwen-Image-2.1-Turbo (convrot.rs:15-68)."""

    def __init__(self, weights: SafetensorsFile):
        self.weights = weights

    @staticmethod
    def open(root: str) -> Optional["ConvRotFile"]:
        """None when the directory holds no ConvRot file (convrot.rs:20-28)."""
        path = os.path.join(root, FILE_NAME)
        if not os.path.isfile(path):
            return None
        return ConvRotFile(SafetensorsFile(path))

    def linear(self, name: str, input: int, output: int, precision: torch.dtype = torch.float16,
               device="cuda") -> "Int8Linear":
        """One projection: ``{name}._weight_qdata`` I8 [output, input],
        ``{name}._weight_scale`` F32 [output], ``{name}._weight_zero_point`` I8
        [output] (convrot.rs:30-67). The int8 rows go to the device as they
        are: their bytes already are the packed words (convrot.rs:151-160)."""
        if input % GROUP or input % 4:
            raise ConfigError(f"{name}: ConvRot input width {input} cannot be rotated in groups of {GROUP}")
        q_shape, codes = self.weights.raw_i8(f"{name}._weight_qdata")
        s_shape, scale = self.weights.raw_f32(f"{name}._weight_scale")
        z_shape, zero = self.weights.raw_i8(f"{name}._weight_zero_point")
        if tuple(q_shape) != (output, input) or scale.size != output or zero.size != output:
            raise ConfigError(f"{name}: ConvRot shapes {list(q_shape)} / scale {list(s_shape)} / "
                              f"zero {list(z_shape)} do not match [{output}, {input}]")
        # host copies out of the read-only map (raw_i8/raw_f32 copy too), then one upload each
        packed = torch.from_numpy(np.array(codes)).to(device).view(torch.int32)
        return Int8Linear(input, output, packed, torch.from_numpy(np.array(scale)).to(device),
                          torch.from_numpy(zero.astype(np.int32)).to(device), precision)


def _is_power_of_four(size: int) -> bool:
    # convrot.rs:135-137
    return size >= 4 and size & (size - 1) == 0 and ((size.bit_length() - 1) % 2 == 0)


def sign_negative(row: int, column: int, size: int) -> bool:
    """H[row][column] < 0: the parity of base-4 digits of ``row ^ column``
    that equal 3 (convrot.rs:139-149, Unsloth ``convrot_hadamard_v1``)."""
    d = row ^ column
    parity = 0
    for _ in range((size.bit_length() - 1) // 2):
        parity ^= int((d & 3) == 3)
        d >>= 2
    return parity == 1


def hadamard(size: int = GROUP) -> np.ndarray:
    """The ``size`` x ``size`` rotation matrix, f32, ``+-2^-(log4 size)``
    (convrot.rs:121-133). Symmetric and its own inverse."""
    if not _is_power_of_four(size):
        raise ValueError("ConvRot group must be a power of four")
    scale = np.float32(2.0 ** -((size.bit_length() - 1) // 2))
    idx = np.arange(size)
    d = idx[:, None] ^ idx[None, :]
    threes = d & (d >> 1) & 0x5555_5555
    parity = np.zeros_like(d)
    for _ in range((size.bit_length() - 1) // 2):
        parity ^= threes & 1
        threes >>= 2
    return np.where(parity == 1, -scale, scale).astype(np.float32)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _float_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return OMNI_F16
    if dtype == torch.float32:
        return OMNI_F32
    raise ValueError(f"unsupported dtype {dtype}")


def convrot_quantize_rows(x: torch.Tensor, group: int = GROUP):
    """Rotate each row's groups of 256 by the Hadamard and quantise the result
    per row (convrot.rs:113-119 then int8_matmul.rs:23-118), in one pass.

    x: [rows, width] f16 or f32 on the GPU, width % 256 == 0 -> (codes int8
    [rows, width], row_scale f32 [rows], row_sum int32 [rows])."""
    if x.dim() != 2:
        raise ValueError("x must be 2-D")
    if x.device.type != "cuda":
        raise _lib.OmniError(_lib.OMNI_BAD_ARGUMENT, "tensors must live on the GPU")
    if x.dtype not in (torch.float16, torch.float32):
        x = x.float()
    if x.stride(1) != 1 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16:
        x = x.contiguous()
    rows, width = x.shape
    words = torch.empty((rows, width // 4), dtype=torch.int32, device=x.device)
    scale = torch.empty(rows, dtype=torch.float32, device=x.device)
    total = torch.empty(rows, dtype=torch.int32, device=x.device)
    st = _lib.check(_lib.lib().omni_convrot_quantize_rows(
        _ptr(x), _float_code(x.dtype), rows, width, x.stride(0), group, _ptr(words), _ptr(scale),
        _ptr(total), _stream(x.device)))
    if st == OMNI_NOT_HANDLED:
        raise ValueError(_lib.last_error())
    return words.view(torch.int8).reshape(rows, width), scale, total


class Int8Linear:
    """One INT8-ConvRot projection (convrot.rs:70-103).

    ``packed`` int32 [output * input / 4] (row-major int8 [output, input],
    4 codes per little-endian word, convrot.rs:151-160), ``scale`` f32
    [output], ``zero`` int32 [output]; ``precision`` is the output dtype
    (torch.float16 for the model's F16, or torch.float32)."""

    def __init__(self, input: int, output: int, packed: torch.Tensor, scale: torch.Tensor,
                 zero: torch.Tensor, precision: torch.dtype = torch.float16):
        if input % GROUP or input % 4:
            # convrot.rs:39-43 refuses such a layer at load time
            raise ValueError(f"ConvRot input width {input} does not split into groups of {GROUP}")
        self.input, self.output = input, output
        self.packed = packed.to(torch.int32).contiguous()
        self.scale = scale.to(torch.float32).contiguous()
        self.zero = zero.to(torch.int32).contiguous()
        self.precision = precision
        _float_code(precision)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [..., input] -> [..., output] in ``precision`` (convrot.rs:81-92)."""
        dims = x.shape
        if dims[-1] != self.input:
            # convrot.rs:84 asserts the width
            raise ValueError(f"ConvRot input width {dims[-1]} != {self.input}")
        rows = int(np.prod(dims[:-1])) if len(dims) > 1 else 1
        flat = x.reshape(rows, self.input)
        if flat.dtype not in (torch.float16, torch.float32):
            flat = flat.float()
        flat = flat.contiguous()
        device = flat.device
        for t in (self.packed, self.scale, self.zero):
            if t.device != device:
                raise _lib.OmniError(_lib.OMNI_BAD_ARGUMENT, "tensors live on different devices")
        L = _lib.lib()
        ws_bytes = L.omni_try_int8_gemm_workspace_size(rows, self.input)
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        out = torch.empty((rows, self.output), dtype=self.precision, device=device)
        st = _lib.check(L.omni_convrot_linear(
            _ptr(flat), _float_code(flat.dtype), rows, self.input, _ptr(self.packed),
            self.packed.numel(), _ptr(self.scale), self.scale.numel(), _ptr(self.zero),
            self.zero.numel(), _ptr(out), _float_code(self.precision), _ptr(workspace), ws_bytes,
            _stream(device)))
        if st == OMNI_NOT_HANDLED:
            # project() expects the op to run (convrot.rs:101 panics on None)
            raise RuntimeError(f"ConvRot int8 gemm: {_lib.last_error()}")
        return out.reshape(*dims[:-1], self.output)

    __call__ = forward
