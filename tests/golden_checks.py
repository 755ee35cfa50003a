"""Checks that pin the oracle. Each returns (ok, message) so the same checks
can be run against a deliberately mutated oracle to show they catch it."""
import json
import os

import numpy as np

import oracle_lib as O

HERE = os.path.dirname(os.path.abspath(__file__))
REF_FIXTURES = os.path.join(HERE, "golden", "reference_fixtures.json")


def load_fixture_tensors(stem):
    with open(REF_FIXTURES) as f:
        data = json.load(f)["files"][stem]["tensors"]
    out = {}
    for name, t in data.items():
        raw = bytes.fromhex(t["hex"])
        dt = {"F8_E4M3": np.uint8, "F8_E5M2": np.uint8, "BF16": np.uint16, "F32": np.float32}[t["dtype"]]
        out[name] = (t["dtype"], t["shape"], np.frombuffer(raw, dtype=dt).copy())
    return out


def f32_bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def check_fp8_unit_kats():
    """crates/ltx-weights/src/fp8.rs:164-205."""
    e4 = lambda b: O.lib().orc_e4m3fn_to_f32(b)
    e5 = lambda b: O.lib().orc_e5m2_to_f32(b)
    conds = [
        (f32_bits(e4(0x00)) == 0x00000000, "e4m3fn 0x00 is +0"),
        (f32_bits(e4(0x80)) == 0x80000000, "e4m3fn 0x80 is -0"),
        (np.isnan(e4(0x7F)) and np.isnan(e4(0xFF)), "e4m3fn 0x7F/0xFF NaN"),
        (abs(e4(0x38) - 1.0) < 1e-6, "e4m3fn 0x38 = 1"),
        (e4(0x77) > 100.0, "e4m3fn 0x77 > 100"),
        (f32_bits(e5(0x00)) == 0, "e5m2 0x00 is +0"),
        (abs(e5(0x3C) - 1.0) < 1e-6, "e5m2 0x3C = 1"),
        (np.isinf(e5(0x7C)) and e5(0x7C) > 0, "e5m2 0x7C = +inf"),
        (np.isinf(e5(0xFC)) and e5(0xFC) < 0, "e5m2 0xFC = -inf"),
    ]
    bad = [m for ok, m in conds if not ok]
    return (not bad, "; ".join(bad))


def check_decode_extremes():
    """Closed-form anchors of the OCP FP8 formats: largest finite value,
    smallest subnormal, smallest normal, and the 1/2/4 ladder."""
    codes = np.arange(256, dtype=np.uint8)
    e4 = O.decode(codes, O.E4M3FN)
    e5 = O.decode(codes, O.E5M2)
    conds = [
        (e4[0x7E] == 448.0, "e4m3fn max finite 448"),
        (e4[0x01] == 2.0 ** -9, "e4m3fn min subnormal 2^-9"),
        (e4[0x08] == 2.0 ** -6, "e4m3fn min normal 2^-6"),
        (e4[0x07] == 7 * 2.0 ** -9, "e4m3fn max subnormal 7*2^-9"),
        (e4[0x40] == 2.0 and e4[0x48] == 4.0, "e4m3fn 2, 4"),
        (e5[0x7B] == 57344.0, "e5m2 max finite 57344"),
        (e5[0x01] == 2.0 ** -16, "e5m2 min subnormal 2^-16"),
        (e5[0x04] == 2.0 ** -14, "e5m2 min normal 2^-14"),
        (e5[0x40] == 2.0 and e5[0x44] == 4.0, "e5m2 2, 4"),
        (all(np.isnan(e5[[0x7D, 0x7E, 0x7F, 0xFD, 0xFE, 0xFF]])), "e5m2 NaN codes"),
    ]
    # sign symmetry and strict monotonicity over the positive finite codes
    fin4 = [b for b in range(0x7F)]
    fin5 = [b for b in range(0x7C)]
    conds.append((np.all(np.diff(e4[fin4]) > 0), "e4m3fn monotone"))
    conds.append((np.all(np.diff(e5[fin5]) > 0), "e5m2 monotone"))
    conds.append((np.array_equal(f32_bits(e4[fin4]) ^ 0x80000000, f32_bits(e4[[b | 0x80 for b in fin4]])), "e4m3fn sign"))
    bad = [m for ok, m in conds if not ok]
    return (not bad, "; ".join(bad))


def check_f16_widening():
    """F16 -> f32 widening (half 2.7.1 `f16::to_f32`, used by store.rs:690-705
    for F16 bases and lora.rs:186-193 for F16 factors) against numpy's
    independent binary16 conversion on all 65536 codes, read as little-endian
    bytes through the oracle's dtype dispatch. Finite codes and infinities
    must match bit for bit; NaN codes must be NaN with numpy's sign and
    payload (mantissa << 13), plus the quiet bit that half's `to_f32` sets."""
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    mine = O.decode(codes, O.F16).view(np.uint32)
    theirs = codes.view(np.float16).astype(np.float32).view(np.uint32)
    nan_c = ((codes & 0x7C00) == 0x7C00) & ((codes & 0x03FF) != 0)
    conds = [
        (np.array_equal(mine[~nan_c], theirs[~nan_c]), "finite codes and infinities differ from numpy"),
        (np.all(np.isnan(mine[nan_c].view(np.float32))), "NaN codes must widen to NaN"),
        (np.array_equal(mine[nan_c] | 0x00400000, theirs[nan_c] | 0x00400000), "NaN sign or payload differs"),
        (np.all(mine[nan_c] & 0x00400000), "widened NaNs must be quiet"),
        (mine[0x0001] == 0x33800000, "smallest subnormal 2^-24"),
        (mine[0x7BFF] == np.float32(65504.0).view(np.uint32), "largest finite 65504"),
    ]
    bad = [m for ok, m in conds if not ok]
    return (not bad, "; ".join(bad))


def check_fp8_fixture():
    """crates/ltx-weights/tests/parity.rs:51-75 with its fixtures; bit-exact."""
    src = load_fixture_tensors("fp8_e4m3fn_parity")
    exp = load_fixture_tensors("fp8_e4m3fn_expected")["w"][2]
    w = src["w"][2].reshape(4, 4)
    scale = src["w_scale"][2]
    got = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, scale)
    same = np.array_equal(f32_bits(got).ravel(), f32_bits(exp))
    return (same, "fp8 fixture differs: got %s want %s" % (got.ravel()[:4], exp[:4]))


def lora_fixture_inputs():
    base = load_fixture_tensors("lora_parity_base")["layer.weight"][2].reshape(8, 4)
    lt = load_fixture_tensors("lora_parity_lora")
    a = lt["layer.lora_A.weight"][2].reshape(2, 4)
    b = lt["layer.lora_B.weight"][2].reshape(8, 2)
    alpha = float(lt["layer.alpha"][2][0])
    exp = load_fixture_tensors("lora_parity_expected")["layer.weight"][2].reshape(8, 4)
    return base, a, b, alpha, exp


def check_lora_fixture():
    """crates/ltx-weights/tests/parity.rs:23-47: bf16 base, f32 rank-2 factors,
    alpha 4, strength 0.75; the f32 chain rounded to bf16 must equal the
    fixture's bf16 tensor bit for bit."""
    base, a, b, alpha, exp = lora_fixture_inputs()
    coeff = O.lora_coeff(0.75, alpha, 2)
    got = O.read_bf16(base, O.BF16, loras=[(b, a, O.F32, coeff)])
    n_same = int(np.sum(got == exp))
    return (n_same == exp.size, "lora fixture: %d/%d bf16 identical" % (n_same, exp.size))


def _f32(v):
    return np.asarray(v, dtype=np.float32)


def check_integration_kats():
    """crates/ltx-weights/tests/integration.rs:399-436 (FP8 with/without scale)
    and :459-586 (LoRA basic, alpha, stacking)."""
    conds = []
    w = np.array([[0x38]], dtype=np.uint8)
    conds.append((O.read_f32(w, O.E4M3FN)[0, 0] == 1.0, "fp8 no scale"))
    conds.append((O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, _f32([3.0]))[0, 0] == 3.0, "fp8 scale 3"))
    eye = _f32([[1, 0], [0, 1]])
    A1, B1 = _f32([[1, 2]]), _f32([[3], [4]])
    got = O.read_f32(eye, O.F32, loras=[(B1, A1, O.F32, O.lora_coeff(1.0, None, 1))])
    conds.append((np.array_equal(got, _f32([[4, 6], [4, 9]])), "lora basic"))
    got = O.read_f32(np.zeros((2, 2), np.float32), O.F32, loras=[(B1, A1, O.F32, O.lora_coeff(1.0, 2.0, 1))])
    conds.append((np.array_equal(got, _f32([[6, 12], [8, 16]])), "lora alpha"))
    A2, B2 = _f32([[1, 0], [0, 1]]), _f32([[2, 0], [0, -2]])
    got = O.read_f32(eye, O.F32, loras=[(B1, A1, O.F32, O.lora_coeff(1.0, None, 1)),
                                        (B2, A2, O.F32, O.lora_coeff(0.5, None, 2))])
    conds.append((np.array_equal(got, _f32([[5, 6], [4, 8]])), "lora stacking"))
    # LoRA on a rectangular weight: B [out x r], A [r x in] with out != in
    Bt, At = _f32([[1], [2], [3]]), _f32([[1, 10]])
    got = O.read_f32(np.zeros((3, 2), np.float32), O.F32, loras=[(Bt, At, O.F32, 1.0)])
    conds.append((np.array_equal(got, _f32([[1, 10], [2, 20], [3, 30]])), "lora rectangular"))
    bad = [m for ok, m in conds if not ok]
    return (not bad, "; ".join(bad))


def random_case(rows, cols, rank, seed, fmt=O.E4M3FN, scale_mode=O.SCALE_ROW, nloras=1):
    rng = np.random.default_rng(seed)
    if fmt == O.E4M3FN:
        codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    else:
        codes = np.array([c for c in range(256) if (c & 0x7F) < 0x7C], dtype=np.uint8)
    w = rng.choice(codes, size=(rows, cols)).astype(np.uint8)
    ns = 1 if scale_mode == O.SCALE_TENSOR else rows
    scales = rng.uniform(1e-3, 1e-1, size=ns).astype(np.float32)
    loras = []
    for l in range(nloras):
        r = rank if l == 0 else max(1, rank // 2)
        b = bf16_rne_np(rng.normal(0, 0.02, size=(rows, r)))
        a = bf16_rne_np(rng.normal(0, 0.02, size=(r, cols)))
        loras.append((b, a, O.BF16, 1.0 if l == 0 else 0.5))
    return w, scales, loras


def bf16_rne_np(x):
    """f64 -> f32 (RNE) -> bf16 (RNE) as uint16, vectorised through the oracle."""
    x32 = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    flat = x32.reshape(1, -1)
    return O.read_bf16(flat, O.F32).reshape(x32.shape)


def check_f32_chain_vs_f64():
    """The f32 chain stays within its forward-error bound of the exact sum:
    |w32 - w64| <= (rank + 2) * 2^-24 * (|deq| + sum |c B A|) elementwise."""
    w, scales, loras = random_case(48, 80, 16, seed=5)
    got = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, scales, loras).astype(np.float64)
    ref = O.read_f64_rows(w, O.E4M3FN, O.SCALE_ROW, scales, loras)
    bound = O.abs_bound_rows(w, O.E4M3FN, O.SCALE_ROW, scales, loras)
    err = np.abs(got - ref)
    lim = (16 + 2) * 2.0 ** -24 * bound
    # the delta must actually matter at this size, or the check is empty
    base_only = O.read_f64_rows(w, O.E4M3FN, O.SCALE_ROW, scales, [])
    moved = np.mean(np.abs(ref - base_only) > 1e-6 * np.abs(ref))
    ok = bool(np.all(err <= lim)) and moved > 0.5
    return (ok, "f32 vs f64: max err/limit %.3g, moved %.2f" % (float(np.max(err / np.maximum(lim, 1e-300))), moved))


def check_row_scale_semantics():
    """Per-row scales (extension): equal row scales reproduce the per-tensor
    path bit for bit; changing scale[o] changes row o only, and row o then
    equals the per-tensor path run with that row's scale."""
    w, scales, loras = random_case(16, 40, 4, seed=9)
    s0 = np.full(16, scales[3], dtype=np.float32)
    t = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, s0[:1], loras)
    r = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, s0, loras)
    ok1 = np.array_equal(f32_bits(t), f32_bits(r))
    s1 = s0.copy()
    s1[5] = np.float32(0.037)
    r1 = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, s1, loras)
    others = [i for i in range(16) if i != 5]
    ok2 = np.array_equal(f32_bits(r1[others]), f32_bits(r[others])) and not np.array_equal(r1[5], r[5])
    t5 = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, s1[5:6], loras)
    ok3 = np.array_equal(f32_bits(r1[5]), f32_bits(t5[5]))
    return (ok1 and ok2 and ok3, "row scale: equal=%s local=%s match=%s" % (ok1, ok2, ok3))


def check_negative_zero_scaled():
    """fma(s, -0, 0) is +0 (store.rs:506); the unscaled path keeps -0."""
    w = np.array([[0x80, 0x00]], dtype=np.uint8)
    scaled = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, _f32([0.5]))
    plain = O.read_f32(w, O.E4M3FN)
    ok = f32_bits(scaled[0, 0]) == 0 and f32_bits(plain[0, 0]) == 0x80000000
    return (bool(ok), "signed zero handling")


ALL_CHECKS = [
    check_fp8_unit_kats,
    check_f16_widening,
    check_decode_extremes,
    check_fp8_fixture,
    check_lora_fixture,
    check_integration_kats,
    check_f32_chain_vs_f64,
    check_row_scale_semantics,
    check_negative_zero_scaled,
]
