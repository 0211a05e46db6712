"""Packed low-bit linear layers for inference.

The reference stores a quantized layer as fake-quantized fp16/bf16 weights
(bigptq.py:278-280).  ``PackedLinear`` keeps the same weights exactly in
3 bits each (2-bit codes, an 8-entry value table per 128-column block
row, one salient-column bitmap per block; the format is described in
include/crbq.h) and multiplies with them directly: up to 16 tokens per call
through the packed GEMV (MFMA on weights decoded in registers), up to 768
through the packed GEMM (each decoded fragment reused for 64 or 128 tokens),
and larger batches, where the product is compute-bound, by unpacking into a
temporary dense weight for the dense GEMM.  The limits are the measured
crossovers on MI355X (4096 x 16384 and 16384 x 4096 fp16 layers).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels

GEMV_MAX_TOKENS = 16
GEMM_MAX_TOKENS = 768


class PackedLinear(nn.Module):
    """nn.Linear with packed weights (in_features = C, out_features = R).
    Buffers: codes, lut, sal (the 3-bit form) and ex_idx, ex_val, ex_delta
    (the rare weights outside their group's table, usually none)."""

    def __init__(self, codes, lut, sal, in_features, bias=None, ex=None):
        super().__init__()
        self.in_features = int(in_features)
        self.out_features = codes.shape[0]
        self.register_buffer("codes", codes)
        self.register_buffer("lut", lut)
        self.register_buffer("sal", sal)
        if ex is None:
            dev = codes.device
            ex = kernels.PackedEx(torch.empty(0, dtype=torch.int64, device=dev),
                                  torch.empty(0, dtype=lut.dtype, device=dev),
                                  torch.empty(0, dtype=torch.float32, device=dev))
        self.register_buffer("ex_idx", ex.idx)
        self.register_buffer("ex_val", ex.val)
        self.register_buffer("ex_delta", ex.delta)
        self.register_buffer("bias", bias)

    @property
    def ex(self) -> kernels.PackedEx:
        return kernels.PackedEx(self.ex_idx, self.ex_val, self.ex_delta)

    @classmethod
    def from_linear(cls, layer: nn.Linear, masks: torch.Tensor) -> "PackedLinear":
        """Pack a quantized nn.Linear given the mask codes its block loop used."""
        codes, lut, sal, ex = kernels.pack(layer.weight.data, masks)
        b = layer.bias.data.clone() if layer.bias is not None else None
        return cls(codes, lut, sal, layer.in_features, b, ex)

    def weight(self) -> torch.Tensor:
        """The dense quantized weight (bit-identical to what was packed)."""
        return kernels.unpack(self.codes, self.lut, self.sal, self.in_features, self.ex)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features)
        if x2.shape[0] <= GEMM_MAX_TOKENS:
            mm = kernels.gemv_packed if x2.shape[0] <= GEMV_MAX_TOKENS else kernels.gemm_packed
            y = mm(self.codes, self.lut, self.sal, self.in_features, x2, self.ex)
            y = y.to(x.dtype)
            if self.bias is not None:
                y = y + self.bias
        else:
            y = F.linear(x2.to(self.lut.dtype), self.weight(), self.bias)
        return y.reshape(*shape[:-1], self.out_features)

    def packed_bytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for t in (self.codes, self.lut, self.sal, self.ex_idx, self.ex_val,
                             self.ex_delta))


def replace_linears(module: nn.Module, packed: dict) -> None:
    """Swap named nn.Linear submodules of module for their PackedLinear."""
    for name, pl in packed.items():
        parent = module
        parts = name.split(".")
        for p in parts[:-1]:
            parent = getattr(parent, p)
        setattr(parent, parts[-1], pl)
