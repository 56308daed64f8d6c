"""Conversions between the oracle's numpy bit patterns and device tensors."""

import numpy as np
import torch


def to_dev(array: np.ndarray, device="cuda") -> torch.Tensor:
    array = np.ascontiguousarray(array)
    if array.dtype == np.uint16:  # BF16 bit patterns
        return torch.from_numpy(array.view(np.int16)).view(torch.bfloat16).to(device)
    return torch.from_numpy(array).to(device)


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def host(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


def randn_bf16(rng: np.random.Generator, shape, scale=1.0) -> np.ndarray:
    from oracle import oracle as O

    return O.f32_to_bf16((rng.standard_normal(shape) * scale).astype(np.float32))


def with_guard(shape, dtype, fill, guard=64, device="cuda"):
    """A contiguous tensor of `shape` inside a buffer with `guard` sentinel elements on
    each side; returns (view, buffer)."""
    numel = int(np.prod(shape))
    buf = torch.full((numel + 2 * guard,), fill, dtype=dtype, device=device)
    return buf[guard : guard + numel].view(*shape), buf


def guard_intact(buf: torch.Tensor, fill, guard=64) -> bool:
    head, tail = buf[:guard], buf[-guard:]
    if isinstance(fill, float) and fill != fill:  # NaN sentinel
        return bool(torch.isnan(head.float()).all() and torch.isnan(tail.float()).all())
    return bool((head == fill).all() and (tail == fill).all())
