"""ltx_weights: MI355X materialisation of ltx-rust's FP8 + LoRA weights.

Python mirror of the `ltx-weights` crate's device path over the C ABI in
include/ltxw.h and include/ltxw_store.h (the library is libltxw.so, built
in-tree for gfx950).
"""
from ._native import (  # noqa: F401
    DESC_EXACT,
    FACTOR_BF16,
    FACTOR_E4M3FN,
    FACTOR_E5M2,
    FACTOR_F16,
    FACTOR_F32,
    FMT_BF16,
    FMT_E4M3FN,
    FMT_E5M2,
    FMT_F16,
    FMT_F32,
    MAX_LORAS,
    NOALLOC_MAX_DESCS,
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
    GateNotScalar,
    QkvSplitDim,
    OutOfMemory,
    UnsupportedDtype,
    WeightError,
    lib,
)
from .store import (  # noqa: F401,E402
    DeviceTensor,
    KeyMap,
    LoraFile,
    MergeReport,
    Scope,
    WeightStore,
)
