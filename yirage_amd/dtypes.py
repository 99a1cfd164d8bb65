"""Element types of the kernel-graph API (python/yirage/_cython/core.pyx:
26-103 of the reference: yr.float16, yr.bfloat16, ...), each carrying the
integer code of yirage::type::DataType (include/yirage/type.h:84-120) that
the C ABI uses and the matching torch dtype."""
from __future__ import annotations

import torch


class dtype:
    SINT_TYPES = ["int8", "int16", "int32", "int64"]
    UINT_TYPES = ["uint8", "uint16", "uint32", "uint64"]
    FP_TYPES = ["fp16", "bf16", "fp32", "fp64"]

    def __init__(self, name: str, code: int, torch_dtype):
        assert name in dtype.SINT_TYPES + dtype.UINT_TYPES + dtype.FP_TYPES, name
        self.name = name
        self.code = code
        self.torch = torch_dtype

    def is_fp16(self):
        return self.name == "fp16"

    def is_bf16(self):
        return self.name == "bf16"

    def is_fp32(self):
        return self.name == "fp32"

    def __eq__(self, other):
        return isinstance(other, dtype) and self.name == other.name

    def __ne__(self, other):
        return not self.__eq__(other)

    def __hash__(self):
        return hash((self.name,))

    def __str__(self):
        return self.name

    __repr__ = __str__

    def __int__(self):
        return self.code


int8 = dtype("int8", 935, torch.int8)
int32 = dtype("int32", 955, torch.int32)
int64 = dtype("int64", 965, torch.int64)
uint8 = dtype("uint8", 936, torch.uint8)
float16 = dtype("fp16", 940, torch.float16)
bfloat16 = dtype("bf16", 941, torch.bfloat16)
float32 = dtype("fp32", 950, torch.float32)
float64 = dtype("fp64", 960, torch.float64)

_BY_CODE = {t.code: t for t in (int8, int32, int64, uint8, float16, bfloat16, float32, float64)}
_BY_TORCH = {t.torch: t for t in (int8, int32, int64, uint8, float16, bfloat16, float32, float64)}


def as_dtype(x) -> dtype:
    """A dtype from a dtype, its integer code or a torch dtype."""
    if isinstance(x, dtype):
        return x
    if isinstance(x, torch.dtype):
        return _BY_TORCH[x]
    return _BY_CODE[int(x)]


def convert_dtype_to_torch_type(t) -> torch.dtype:
    """python/yirage/_cython/core.pyx convert_dtype_to_torch_type."""
    return as_dtype(t).torch
