"""ltx_weights: MI355X materialisation of ltx-rust's FP8 + LoRA weights.

Python mirror of the `ltx-weights` crate's device path over the C ABI in
include/ltxw.h (the library is libltxw.so, built in-tree for gfx950).
"""
from ._native import (  # noqa: F401
    FMT_E4M3FN,
    FMT_E5M2,
    MAX_LORAS,
    OUT_BF16,
    OUT_F32,
    SCALE_NONE,
    SCALE_ROW,
    SCALE_TENSOR,
    Context,
    DeviceError,
    DuplicateKey,
    InvalidArgument,
    InvalidTensorData,
    IoError,
    LoraRankMismatch,
    LoraShapeMismatch,
    MissingKey,
    NoLoraMatches,
    OutOfMemory,
    UnsupportedDtype,
    WeightError,
    lib,
)
