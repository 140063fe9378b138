# SPDX-License-Identifier: Apache-2.0
# The operator names, signatures, argument checks and error texts here follow snowllm/ops/_common.py
# (SPDX-FileCopyrightText: Copyright contributors to the SnowLLM project), which this
# module keeps so that the reference's callers can use it unchanged.
"""Operator plumbing shared by the wrappers (mirrors snowllm/ops/_common.py:48-100).

Tensors are validated before every call -- device, dtype, shape and layout -- and raw
data pointers plus torch's current HIP stream are handed to the C ABI.
"""
import torch

from . import _capi
from .errors import SnowLLMError

_capi.assert_single_hip_runtime()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _p(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def _chk(t: torch.Tensor, name: str, dtype: torch.dtype, *shape: int) -> None:
    if t.dtype != dtype:
        raise SnowLLMError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise SnowLLMError(f"{name}: expected a CUDA tensor, got {t.device}")
    if not t.is_contiguous():
        raise SnowLLMError(f"{name}: must be contiguous")
    if shape and tuple(t.shape) != shape:
        raise SnowLLMError(f"{name}: expected shape {shape}, got {tuple(t.shape)}")


def _chk_rows(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    if t.dtype != dtype:
        raise SnowLLMError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise SnowLLMError(f"{name}: expected a CUDA tensor, got {t.device}")
    if t.dim() != 2 or t.stride(1) != 1:
        raise SnowLLMError(f"{name}: must be a 2-D row-strided tensor, got shape "
                           f"{tuple(t.shape)} stride {t.stride()}")


def empty(*shape, dtype, device="cuda") -> torch.Tensor:
    return torch.empty(*shape, dtype=dtype, device=device)


def empty_bytes(n: int) -> torch.Tensor:
    return torch.empty(int(n), dtype=torch.uint8, device="cuda")


def synchronize() -> None:
    _capi.synchronize(_stream())
