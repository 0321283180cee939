"""Batched token sampling on the GPU (reference: qwen3/sampling.py).

sample_tokens keeps the reference's signature and contract: logits (B, V),
temperature / top_k / top_p as scalars or per-row lists / tensors, returns
(B, 1) int64.  Rows with temperature <= 0 take the argmax; the rest draw from
softmax(logits / temperature) restricted to the top_k largest logits (all
when top_k <= 0) and, within them, to the leading tokens whose mass before
them is <= top_p.  The rows go through the sampling kernels
(qwen3_sample_ws_bf16: for batches of up to 128 rows two launches that
split each row over 2-8 workgroups, else one workgroup per row), or, when
all rows are greedy and the batch is larger, the argmax kernel; there is no
host round trip for per-row parameters given as device tensors.  The random
stream is the kernel's own (Philox4x32-10), so draws match the reference in
distribution, not token for token — as the reference's own Triton path does
against its torch path (qwen3/sampling.py:17-20).
"""
from __future__ import annotations

import torch

from . import _lib
from .kernels.model_ops import argmax

__all__ = ["sample_tokens"]

_SEED_COUNTER = 0


def _next_seed() -> int:
    """A fresh seed per call when none is given (the reference's rule of a
    counter over torch.initial_seed(), qwen3/sampling.py:44-47)."""
    global _SEED_COUNTER
    _SEED_COUNTER += 1
    return (torch.initial_seed() + _SEED_COUNTER * 0x9E3779B1) & 0xFFFFFFFFFFFF


def _param(value, B: int, device, dtype) -> torch.Tensor:
    if isinstance(value, torch.Tensor):
        t = value.to(device=device, dtype=dtype)
        if t.ndim == 0:
            t = t.expand(B)
        return t.reshape(B).contiguous()
    if isinstance(value, (list, tuple)):
        return torch.tensor(value, device=device, dtype=dtype)
    return torch.full((B,), value, device=device, dtype=dtype)


def _all_greedy(temperature) -> bool:
    if isinstance(temperature, torch.Tensor):
        return temperature.device.type == "cpu" and bool((temperature <= 0).all())
    if isinstance(temperature, (list, tuple)):
        return all(float(t) <= 0 for t in temperature)
    return float(temperature) <= 0


_WORKSPACES: dict = {}
# Workspaces replaced by a larger one stay allocated until the process ends:
# a graph captured earlier holds the old address and may still be replayed.
_SUPERSEDED: list = []


def _workspace(dev, stream: int, B: int, V: int):
    """The parallel form's workspace for this device and stream (grown, never
    shrunk, never freed); None under graph capture when it would have to grow
    (the call then takes the single-workgroup form, which needs none)."""
    need = int(_lib.load().qwen3_sample_workspace_bytes(B, V))
    if need == 0:  # one part per row: the single-workgroup form
        return None
    key = (str(dev), stream)
    ws = _WORKSPACES.get(key)
    if ws is not None and ws.numel() >= need:
        return ws
    if torch.cuda.is_current_stream_capturing():
        return None
    if ws is not None:
        _SUPERSEDED.append(ws)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    _WORKSPACES[key] = ws
    return ws


def sample_tokens(logits: torch.Tensor, temperature=0.0, top_k=0, top_p=1.0,
                  seed: int | None = None) -> torch.Tensor:
    """(B, V) bf16 logits -> (B, 1) int64 tokens (reference:
    qwen3/sampling.py:234-270)."""
    if logits.ndim != 2:
        raise ValueError(f"logits must be (B, V), got shape {tuple(logits.shape)}")
    assert logits.dtype == torch.bfloat16 and logits.stride(1) == 1
    B, V = logits.shape
    dev = _lib.require_hip(logits)
    stream = _lib.stream_of(dev)
    if _all_greedy(temperature):
        ws = _workspace(dev, stream, B, V)
        if ws is None:  # one workgroup per row: the argmax kernel
            return argmax(logits).view(B, 1)
        # a small batch: the parallel form's greedy path (no temperatures:
        # every row greedy), each row split over several workgroups
        out = torch.empty(B, dtype=torch.int64, device=dev)
        _lib.check(_lib.load().qwen3_sample_ws_bf16(
            logits.data_ptr(), logits.stride(0), B, V, None, None, None, 0, out.data_ptr(),
            ws.data_ptr(), ws.numel(), stream), "qwen3_sample_ws_bf16")
        return out.view(B, 1)
    t = _param(temperature, B, dev, torch.float32)
    k = _param(top_k, B, dev, torch.int32)
    p = _param(top_p, B, dev, torch.float32)
    if seed is None:
        seed = _next_seed()
    out = torch.empty(B, dtype=torch.int64, device=dev)
    ws = _workspace(dev, stream, B, V)
    rc = _lib.load().qwen3_sample_ws_bf16(
        logits.data_ptr(), logits.stride(0), B, V, t.data_ptr(), k.data_ptr(), p.data_ptr(),
        int(seed) & (2 ** 64 - 1), out.data_ptr(), None if ws is None else ws.data_ptr(),
        0 if ws is None else ws.numel(), stream)
    _lib.check(rc, "qwen3_sample_ws_bf16")
    return out.view(B, 1)
