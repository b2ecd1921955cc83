"""Device-tensor plumbing shared by the host modules (torch is used for device
memory and streams only; every computation runs in libtorque_hip)."""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from torque_hip._lib import TQ_F16, TQ_F32


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("torque_hip needs a HIP device (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def stream_handle(dev: torch.device | None = None) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _aligned(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def to_device(values: Any, dev: torch.device, *, keep_f16: bool = True) -> torch.Tensor:
    """Contiguous, 16-byte aligned device tensor, float32 (float16 kept when allowed)."""
    if isinstance(values, torch.Tensor):
        t = values
        if t.dtype not in (torch.float32, torch.float16) or (t.dtype == torch.float16 and not keep_f16):
            t = t.to(torch.float32)
        t = t.to(dev).contiguous()
    else:
        array = np.asarray(values)
        if array.dtype == np.float16 and keep_f16:
            t = torch.from_numpy(np.ascontiguousarray(array)).to(dev)
        else:
            t = torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(dev)
    if not _aligned(t):
        t = t.clone()
    return t


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float16:
        return TQ_F16
    if t.dtype == torch.float32:
        return TQ_F32
    raise ValueError(f"unsupported dtype {t.dtype}")


def codes_to_device(values: Any, dev: torch.device) -> torch.Tensor:
    """uint32 packed codes as a contiguous device int32 view (same bits)."""
    if isinstance(values, torch.Tensor):
        t = values
        if t.dtype == torch.uint32:
            t = t.view(torch.int32)
        elif t.dtype != torch.int32:
            t = t.to(torch.int64).to(torch.int32)
        t = t.to(dev).contiguous()
    else:
        t = torch.from_numpy(np.ascontiguousarray(np.asarray(values, dtype=np.uint32)).view(np.int32)).to(dev)
    if not _aligned(t):
        t = t.clone()
    return t


def codes_to_numpy(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().view(np.uint32)


def shape_of(values: Any) -> tuple[int, ...]:
    if isinstance(values, torch.Tensor):
        return tuple(int(s) for s in values.shape)
    return tuple(np.shape(values))
