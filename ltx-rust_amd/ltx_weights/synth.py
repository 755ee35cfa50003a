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
