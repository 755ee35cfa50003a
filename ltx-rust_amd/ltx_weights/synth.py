"""Seeded synthetic inputs in the shapes of the weight-materialisation workloads.

Distributions:
  - FP8 weights: bytes uniform over the non-NaN codes of the format (254 for
    e4m3fn; 248 for e5m2, Inf excluded unless asked for).
  - Scales: f32 uniform on [1e-3, 1e-1], one per tensor or one per output row.
  - LoRA factors: N(0, 0.02^2) drawn in f64 and rounded to bf16 (RNE).

Shapes follow one LTX-2.5 DiT block: attention q/k/v/o and cross-attention
q/k/v/o are 4096 x 4096, FFN up is 16384 x 4096, FFN down is 4096 x 16384.
"""
import numpy as np

E4M3FN, E5M2 = 0, 1
SCALE_NONE, SCALE_TENSOR, SCALE_ROW = 0, 1, 2

E4M3FN_CODES = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
E5M2_FINITE_CODES = np.array([c for c in range(256) if (c & 0x7F) < 0x7C], dtype=np.uint8)

# (name, out_features, in_features) of one DiT block's LoRA-targeted linears.
BLOCK_LINEARS = [
    ("attn1.to_q", 4096, 4096),
    ("attn1.to_k", 4096, 4096),
    ("attn1.to_v", 4096, 4096),
    ("attn1.to_out.0", 4096, 4096),
    ("attn2.to_q", 4096, 4096),
    ("attn2.to_k", 4096, 4096),
    ("attn2.to_v", 4096, 4096),
    ("attn2.to_out.0", 4096, 4096),
    ("ff.net.0.proj", 16384, 4096),
    ("ff.net.2", 4096, 16384),
]


def bf16_from_f64(x):
    """Round f64 to bf16 (round-to-nearest-even on 8 significant bits), as uint16."""
    x = np.asarray(x, dtype=np.float64)
    m, e = np.frexp(x)
    q = np.rint(m * 256.0)  # rint rounds half to even
    v = np.ldexp(q / 256.0, e).astype(np.float32)  # exact: 8 significant bits
    return (v.view(np.uint32) >> 16).astype(np.uint16)


def fp8_weights(rng, rows, cols, fmt=E4M3FN):
    codes = E4M3FN_CODES if fmt == E4M3FN else E5M2_FINITE_CODES
    idx = rng.integers(0, len(codes), size=(rows, cols), dtype=np.uint16)
    return codes[idx]


def scales(rng, rows, mode):
    if mode == SCALE_NONE:
        return None
    n = 1 if mode == SCALE_TENSOR else rows
    return rng.uniform(1e-3, 1e-1, size=n).astype(np.float32)


def lora_factors(rng, rows, cols, rank, std=0.02):
    """(B [rows x rank], A [rank x cols]) as bf16 bit patterns."""
    b = bf16_from_f64(rng.normal(0.0, std, size=(rows, rank)))
    a = bf16_from_f64(rng.normal(0.0, std, size=(rank, cols)))
    return b, a


def tensor_case(seed, rows, cols, fmt=E4M3FN, scale_mode=SCALE_ROW, loras=((64, 1.0),)):
    """One tensor: dict(w, scales, loras=[(B, A, rank, coeff)], ...)."""
    rng = np.random.default_rng(seed)
    w = fp8_weights(rng, rows, cols, fmt)
    s = scales(rng, rows, scale_mode)
    ls = []
    for rank, coeff in loras:
        b, a = lora_factors(rng, rows, cols, rank)
        ls.append((b, a, rank, float(coeff)))
    return {"w": w, "scales": s, "loras": ls, "rows": rows, "cols": cols, "fmt": fmt,
            "scale_mode": scale_mode}


def algorithmic_bytes(rows, cols, scale_mode, ranks, out_bytes=2):
    """FP8 in + output + scales + bf16 factors, each read or written once."""
    sb = 0 if scale_mode == SCALE_NONE else (4 if scale_mode == SCALE_TENSOR else 4 * rows)
    return rows * cols * (1 + out_bytes) + sb + sum(2 * r * (rows + cols) for r in ranks)


def lora_flops(rows, cols, ranks):
    return sum(2 * rows * cols * r for r in ranks)


# ---------------------------------------------------------------------------
# Counter-based generator of the synthetic checkpoint files (the numpy
# statement of ltx-rust_amd/synth/synth_writer.cpp): every value is a pure
# function of (seed, tensor name, element index), so sampled rows of a
# multi-GB file can be regenerated here to check a materialised result.
# ---------------------------------------------------------------------------
import ctypes  # noqa: E402
import os  # noqa: E402

_U64 = np.uint64
_GOLDEN = _U64(0x9E3779B97F4A7C15)
_SYNTH_LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "_build",
                          "libltxw_synth.so")
KIND_E4M3FN, KIND_E5M2, KIND_F32_SCALE, KIND_BF16 = 0, 1, 2, 3


def _mix(x):
    x = x ^ (x >> _U64(30))
    x = x * _U64(0xBF58476D1CE4E5B9)
    x = x ^ (x >> _U64(27))
    x = x * _U64(0x94D049BB133111EB)
    return x ^ (x >> _U64(31))


def _fnv1a64(name):
    h = 0xCBF29CE484222325
    for c in name.encode():
        h = ((h ^ c) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_key(seed, name):
    with np.errstate(over="ignore"):
        return _mix(_U64(seed) ^ _mix(np.array([_fnv1a64(name)], dtype=_U64)))[0]


def _words(key, idx):
    idx = np.asarray(idx, dtype=_U64)
    with np.errstate(over="ignore"):
        return _mix(key + (idx + _U64(1)) * _GOLDEN)


def gen_fp8(seed, name, elem_idx, fmt=E4M3FN):
    """FP8 bytes at flat element indices `elem_idx` of tensor `name`."""
    e = np.asarray(elem_idx, dtype=_U64)
    w = _words(tensor_key(seed, name), e >> _U64(3))
    b = ((w >> ((e & _U64(7)) * _U64(8))) & _U64(0xFF)).astype(np.uint32)
    codes = E4M3FN_CODES if fmt == E4M3FN else E5M2_FINITE_CODES
    return codes[(b * np.uint32(len(codes))) >> np.uint32(8)]


def gen_scales(seed, name, n):
    u = (_words(tensor_key(seed, name), np.arange(n, dtype=_U64)) >> _U64(11)).astype(np.float64) * 2.0 ** -53
    return (1e-3 + u * (0.1 - 1e-3)).astype(np.float32)


def _bf16_rne_f32(f):
    u = np.asarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def gen_bf16(seed, name, elem_idx):
    """bf16 bit patterns of the N(0, 0.02^2) factors at flat element indices."""
    e = np.asarray(elem_idx, dtype=_U64)
    key = tensor_key(seed, name)
    total = np.zeros(e.shape, dtype=np.uint64)
    for q in range(3):
        w = _words(key, e * _U64(3) + _U64(q))
        for lane in range(4):
            total += (w >> _U64(16 * lane)) & _U64(0xFFFF)
    z = total.astype(np.float64) / 65536.0 - 6.0
    return _bf16_rne_f32((0.02 * z).astype(np.float32))


# Edge tensors of the mixed-format set: (name, out, in).
EDGE_LINEARS = [("edge.proj_a", 4096, 4104), ("edge.proj_b", 4104, 16384)]
CKPT_PREFIX = "model.diffusion_model."


def model_layout(n_blocks, variant):
    """[(store key, fmt, scale_mode, out, in)] of a synthetic model file, in
    file order (store keys are the names after the checkpoint prefix)."""
    out = []
    for b in range(n_blocks):
        for nm, r, c in BLOCK_LINEARS:
            ffn = nm.startswith("ff.")
            if variant == 0:
                fmt, sm = E4M3FN, SCALE_ROW
            else:
                fmt, sm = (E5M2, SCALE_ROW) if ffn else (E4M3FN, SCALE_TENSOR)
            out.append((f"transformer_blocks.{b}.{nm}.weight", fmt, sm, r, c))
    if variant == 1:
        out.append(("edge.proj_a.weight", E4M3FN, SCALE_TENSOR, 4096, 4104))
        out.append(("edge.proj_b.weight", E5M2, SCALE_ROW, 4104, 16384))
    return out


_synth = None


def synth_lib():
    global _synth
    if _synth is None:
        if not os.path.exists(_SYNTH_LIB):
            raise ImportError(f"libltxw_synth.so is not built: {_SYNTH_LIB}")
        L = ctypes.CDLL(_SYNTH_LIB)
        L.ltxs_write_model.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.ltxs_write_lora.argtypes = [ctypes.c_char_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_int]
        _synth = L
    return _synth


def write_model(path, seed, n_blocks, variant=0, threads=8):
    rc = synth_lib().ltxs_write_model(str(path).encode(), seed, n_blocks, variant, threads)
    if rc != 0:
        raise OSError(f"writing {path} failed ({rc})")


def write_lora(path, seed, n_blocks, rank, variant=0, threads=8):
    rc = synth_lib().ltxs_write_lora(str(path).encode(), seed, n_blocks, variant, rank, threads)
    if rc != 0:
        raise OSError(f"writing {path} failed ({rc})")


def model_rows(seed, key, fmt, scale_mode, rows_sel, cols, n_rows):
    """Regenerated (FP8 rows, scales) of one model tensor: bytes [len(rows_sel), cols]
    and the f32 scales the store applies (per row, or the one scale)."""
    name = CKPT_PREFIX + key
    rows_sel = np.asarray(rows_sel, dtype=np.uint64)
    idx = rows_sel[:, None] * np.uint64(cols) + np.arange(cols, dtype=np.uint64)[None, :]
    w = gen_fp8(seed, name, idx, fmt)
    if scale_mode == SCALE_ROW:
        s = gen_scales(seed, name + "_scale", n_rows)
    else:
        s = gen_scales(seed, name + "_scale", 1)
    return w, s


def lora_factors_rows(seed, key, rank, rows_sel, rows, cols):
    """(B rows [len(rows_sel), rank], A [rank, cols]) bf16 patterns of one LoRA file's factors."""
    prefix = key[: -len(".weight")]
    rows_sel = np.asarray(rows_sel, dtype=np.uint64)
    bidx = rows_sel[:, None] * np.uint64(rank) + np.arange(rank, dtype=np.uint64)[None, :]
    b = gen_bf16(seed, prefix + ".lora_B.weight", bidx)
    a = gen_bf16(seed, prefix + ".lora_A.weight", np.arange(rank * cols, dtype=np.uint64).reshape(rank, cols))
    return b, a
