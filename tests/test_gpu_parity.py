"""GPU parity: the HIP path through the C ABI against the CPU oracle.

Bars: dequantisation is bit-exact in bf16 and f32 (NaN encodings included);
the fused LoRA merge follows the tolerance in gpu_util.compare_lora_bf16
(1 bf16 ulp, an f32-error escape for ill-conditioned elements, Frobenius
<= 1e-3 against the bf16-rounded f64 oracle). The generic kernel follows the
reference's operation order and must be bit-exact.
"""
import sys

import numpy as np
import pytest

import gpu_util as U
import ltx_weights as lw
from ltx_weights import synth

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ctx():
    c = lw.Context(0)
    yield c
    c.close()


def run_case(ctx, case, out_dtype=lw.OUT_BF16, **kw):
    d = U.Dev(ctx, case, out_dtype, **kw)
    try:
        d.run()
        return d.result()
    finally:
        d.free()


def all_codes_case(fmt, scale_mode, rows=64, cols=256, with_inf=True, loras=()):
    """Every byte value in every row, rotated per row."""
    w = np.array([np.roll(np.arange(256, dtype=np.uint8), r) for r in range(rows)])[:, :cols]
    rng = np.random.default_rng(77)
    return {"w": np.ascontiguousarray(w), "scales": synth.scales(rng, rows, scale_mode), "loras": list(loras),
            "rows": rows, "cols": cols, "fmt": fmt, "scale_mode": scale_mode}


@pytest.mark.parametrize("fmt", [lw.FMT_E4M3FN, lw.FMT_E5M2])
@pytest.mark.parametrize("scale_mode", [lw.SCALE_NONE, lw.SCALE_TENSOR, lw.SCALE_ROW])
@pytest.mark.parametrize("out_dtype", [lw.OUT_BF16, lw.OUT_F32])
def test_dequant_all_codes_bit_exact(ctx, fmt, scale_mode, out_dtype):
    log("case: all codes", fmt, scale_mode, out_dtype)
    case = all_codes_case(fmt, scale_mode)
    got = run_case(ctx, case, out_dtype)
    ref = U.oracle_bf16(case) if out_dtype == lw.OUT_BF16 else U.oracle_f32(case)
    assert np.array_equal(got.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32),
                          ref.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32))


def test_dequant_4096_per_tensor_scale_bit_exact(ctx):
    """4096 x 4096 e4m3fn with one f32 scale from U[1e-3, 1e-1], bf16 out."""
    log("case: dequant 4096x4096 tensor scale")
    case = synth.tensor_case(1001, 4096, 4096, synth.E4M3FN, synth.SCALE_TENSOR, loras=())
    got = run_case(ctx, case)
    ref = U.oracle_bf16(case)
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape", [(1, 1), (3, 17), (7, 4104), (129, 33), (2, 8), (5, 15), (1, 4097), (64, 16)])
@pytest.mark.parametrize("scale_mode", [lw.SCALE_NONE, lw.SCALE_TENSOR, lw.SCALE_ROW])
def test_dequant_ragged_shapes_bit_exact(ctx, shape, scale_mode):
    log("case: ragged", shape, scale_mode)
    case = synth.tensor_case(7, shape[0], shape[1], synth.E5M2, scale_mode, loras=())
    got = run_case(ctx, case)
    assert np.array_equal(got, U.oracle_bf16(case))


@pytest.mark.parametrize("shape", [(65, 4096), (200, 4104), (127, 136), (63, 8)])
@pytest.mark.parametrize("fmt", [synth.E4M3FN, synth.E5M2])
def test_dequant_partial_row_tiles_row_scales(ctx, shape, fmt):
    """The tiled kernel takes 64 rows x 128 columns per workgroup: row counts
    off a multiple of 64 (a last tile of 1, 8 or 63 rows) and a last band
    of 8 columns, with one scale per row, in both output types."""
    log("case: partial row tiles", shape, fmt)
    case = synth.tensor_case(11, shape[0], shape[1], fmt, synth.SCALE_ROW, loras=())
    for out_dtype in (lw.OUT_BF16, lw.OUT_F32):
        got = run_case(ctx, case, out_dtype)
        ref = U.oracle_bf16(case) if out_dtype == lw.OUT_BF16 else U.oracle_f32(case)
        assert np.array_equal(got.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32),
                              ref.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32)), out_dtype


@pytest.mark.parametrize("w_offset,out_offset", [(1, 0), (0, 2), (3, 6), (8, 0)])
def test_dequant_unaligned_pointers_bit_exact(ctx, w_offset, out_offset):
    log("case: unaligned", w_offset, out_offset)
    case = synth.tensor_case(8, 33, 100, synth.E4M3FN, synth.SCALE_ROW, loras=())
    got = run_case(ctx, case, w_offset=w_offset, out_offset=out_offset)
    assert np.array_equal(got, U.oracle_bf16(case))


def test_fused_4096_rank64_row_scale(ctx):
    """4096 x 4096 e4m3fn, per-row scales, rank-64 bf16 LoRA, alpha = 1."""
    log("case: fused 4096x4096 r64")
    case = synth.tensor_case(1002, 4096, 4096, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
    got = run_case(ctx, case)
    stats = U.compare_lora_bf16(case, got)
    log("stats", stats)


@pytest.mark.parametrize("rows,cols,ranks,fmt,scale_mode", [
    (4104, 512, ((64, 1.0),), synth.E4M3FN, synth.SCALE_ROW),      # row tail
    (256, 4104, ((64, 1.0),), synth.E4M3FN, synth.SCALE_TENSOR),   # column tail (4104 = 8 mod 16)
    (130, 264, ((16, 0.5),), synth.E5M2, synth.SCALE_ROW),
    (96, 136, ((8, 2.0),), synth.E4M3FN, synth.SCALE_NONE),
    (200, 384, ((128, 0.5),), synth.E4M3FN, synth.SCALE_ROW),      # two K passes
    (300, 520, ((32, 1.0), (128, 0.5)), synth.E5M2, synth.SCALE_ROW),   # stacked LoRAs
    (128, 128, ((64, 1.0), (8, -0.25), (16, 0.75)), synth.E4M3FN, synth.SCALE_TENSOR),
    (1, 8, ((8, 1.0),), synth.E4M3FN, synth.SCALE_ROW),
])
def test_fused_shapes(ctx, rows, cols, ranks, fmt, scale_mode):
    log("case: fused", rows, cols, ranks, fmt, scale_mode)
    case = synth.tensor_case(rows * 31 + cols, rows, cols, fmt, scale_mode, loras=ranks)
    got = run_case(ctx, case)
    U.compare_lora_bf16(case, got)


@pytest.mark.parametrize("coeffs", [(0.5, 1e-6, 4.0), (-3.0, 1e4, 2.0 ** -20), (1.0, 1.0, -1.0)])
def test_fused_several_loras_coefficient_ratios(ctx, coeffs):
    """Several LoRAs share one accumulator rescaled by c_l / c_(l+1) between
    them; large and small ratios and equal coefficients stay within tolerance."""
    log("case: fused ratios", coeffs)
    ranks = tuple(zip((32, 64, 8), coeffs))
    case = synth.tensor_case(4242, 300, 264, synth.E4M3FN, synth.SCALE_ROW, loras=ranks)
    got = run_case(ctx, case)
    U.compare_lora_bf16(case, got)


@pytest.mark.parametrize("coeffs", [(1.0, 0.0), (2.0 ** -30, 1.0), (1.0, 2.0 ** 40), (3.0, -(2.0 ** 25))])
def test_several_loras_extreme_coefficients_use_reference_order(ctx, coeffs):
    """A zero or extreme coefficient next to another LoRA is routed to the
    reference-order kernel (no rescaling by c_l / c_(l+1)), so the
    result is the oracle's bit for bit."""
    log("case: extreme coefficients", coeffs)
    ranks = tuple(zip((32, 128), coeffs))
    case = synth.tensor_case(4343, 300, 520, synth.E5M2, synth.SCALE_ROW, loras=ranks)
    got = run_case(ctx, case)
    assert np.array_equal(got.view(np.uint16), U.oracle_bf16(case).view(np.uint16))


def factor_codes(rng, fdt, shape):
    """Factor elements of type fdt with magnitudes below 1/8: f16 from
    N(0, 0.02^2); FP8 codes with small exponent fields, both signs, zeros and
    subnormals included."""
    if fdt == lw.FACTOR_F16:
        return rng.normal(0.0, 0.02, size=shape).astype(np.float16).view(np.uint16)
    exp_bits, man_bits, e_max = (4, 3, 4) if fdt == lw.FACTOR_E4M3FN else (5, 2, 12)
    e = rng.integers(0, e_max + 1, size=shape)
    m = rng.integers(0, 1 << man_bits, size=shape)
    sgn = rng.integers(0, 2, size=shape)
    return ((sgn << 7) | (e << man_bits) | m).astype(np.uint8)


@pytest.mark.parametrize("fdt", [lw.FACTOR_F16, lw.FACTOR_E4M3FN, lw.FACTOR_E5M2])
@pytest.mark.parametrize("ranks,shape", [(((64, 1.0),), (300, 520)), (((32, 1.0), (128, 0.5)), (257, 4104)),
                                         (((8, 2.0), (16, -0.75), (40, 1.25)), (64, 136))])
def test_fused_non_bf16_factors(ctx, fdt, ranks, shape):
    """f16 factors on the f16 MFMA, FP8 factors widened to bf16 (exact) on the
    bf16 MFMA: within the fused path's tolerance of the oracle, which widens
    them as lora.rs:176-209 does; with LTXW_DESC_EXACT, bit-exact."""
    log("case: factor type", fdt, ranks, shape)
    rows, cols = shape
    rng = np.random.default_rng(fdt * 1000 + rows)
    case = synth.tensor_case(rows + cols + fdt, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=())
    case["loras"] = [(factor_codes(rng, fdt, (rows, r)), factor_codes(rng, fdt, (r, cols)), r, c, fdt) for r, c in ranks]
    got, = run_grouped(ctx, [case])
    U.compare_lora_bf16(case, got)
    exact, = run_grouped(ctx, [case], flags=lw.DESC_EXACT)
    assert np.array_equal(exact, U.oracle_bf16(case))


@pytest.mark.parametrize("kind", ["r64", "r128", "r32+r128", "r64 f16 factors", "r64 bf16 base", "r128 f32 out",
                                  "r128 ragged", "r32+r128 ragged"])
def test_large_launch_b_fragment_swap_bit_identical(ctx, kind):
    """Launches of 1024 workgroups and more load the LoRA B fragments of a
    K-step pair swapped on odd rows when a LoRA's row is a multiple of 128
    bytes (ranks 64 and 128 here). Same data, same arithmetic: six copies of
    one 4096 x 4096 tensor in one grouped launch (6 x 512 workgroups) equal the
    tensor launched alone (512, no swap) bit for bit, and the tensor is within
    the fused tolerance of the oracle on sampled rows. The ragged kinds take
    4104 x 4104 (6 x 561 workgroups, partial tiles at the row and column ends)."""
    log("case: B-fragment swap", kind)
    rows = cols = 4104 if kind.endswith("ragged") else 4096
    kind = kind.replace(" ragged", "")
    rng = np.random.default_rng(4096)
    if kind == "r64 bf16 base":
        case = {"w": synth.bf16_from_f64(rng.normal(0.0, 0.05, size=(rows, cols))), "scales": None, "rows": rows,
                "cols": cols, "fmt": lw.FMT_BF16, "scale_mode": lw.SCALE_NONE, "loras": []}
        b, a = synth.lora_factors(rng, rows, cols, 64)
        case["loras"] = [(b, a, 64, 1.0)]
    else:
        ranks = {"r64": ((64, 1.0),), "r128": ((128, 0.5),), "r32+r128": ((32, 1.0), (128, 0.5)),
                 "r64 f16 factors": (), "r128 f32 out": ((128, 0.5),)}[kind]
        case = synth.tensor_case(4097, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=ranks)
        if kind == "r64 f16 factors":
            case["loras"] = [(factor_codes(rng, lw.FACTOR_F16, (rows, 64)), factor_codes(rng, lw.FACTOR_F16, (64, cols)),
                              64, 1.0, lw.FACTOR_F16)]
    out_dtype = lw.OUT_F32 if kind.endswith("f32 out") else lw.OUT_BF16
    d = U.Dev(ctx, case, out_dtype)
    outs = []
    try:
        d.run()
        alone = d.result()
        sel = np.unique(np.concatenate([[0, 1, rows - 1], rng.choice(rows, 40, replace=False)]))
        if out_dtype == lw.OUT_BF16:
            U.compare_lora_bf16(case, alone[sel], row_sel=sel)
        else:  # the f32 forward-error bound of both summation orders
            import oracle_lib as O
            w, f, m, sc, loras = U.oracle_args(case, sel)
            bound = O.abs_bound_rows(w, f, m, sc, loras)
            err = np.abs(alone[sel].astype(np.float64) - U.oracle_f32(case, sel).astype(np.float64))
            assert np.all(err <= 2 * (128 + 4) * 2.0 ** -24 * bound)
        outs = [ctx.alloc(rows * cols * d.ob) for _ in range(6)]
        ctx.grouped([{"w": d.w, "out": o, "scales": d.s, "rows": rows, "cols": cols, "fmt": case["fmt"],
                      "scale_mode": case["scale_mode"], "out_dtype": out_dtype, "loras": d.loras} for o in outs])
        for o in outs:
            got = np.empty_like(alone)
            ctx.download(o, got)
            assert np.array_equal(got.view(np.uint8), alone.view(np.uint8))
    finally:
        for o in outs:
            ctx.free(o)
        d.free()


@pytest.mark.parametrize("ranks", [((64, 1.0),), ((32, 1.0), (128, 0.5))])
@pytest.mark.parametrize("copies", [1, 6])
def test_zero_lora_equals_dequant_at_full_size(ctx, ranks, copies):
    """A size-independent property at the full 4096 x 4096 size: with every B
    factor zero the LoRA product is +0, and the fused epilogue
    fma(scale, decode(w), coeff * 0) is the dequantisation fma(scale, decode(w), 0)
    bit for bit (row scales, so -0 turns +0 on both sides). Covers every
    element's index mapping in the fused kernels' epilogue; six copies in one
    grouped launch take the B-fragment pair swap."""
    log("case: zero LoRA", ranks, copies)
    case = synth.tensor_case(4444, 4096, 4096, synth.E4M3FN, synth.SCALE_ROW, loras=ranks)
    case["loras"] = [(np.zeros_like(b), a, r, c) for (b, a, r, c) in case["loras"]]
    d = U.Dev(ctx, case)
    outs = []
    try:
        if copies == 1:
            d.run()
            got = [d.result()]
        else:
            outs = [ctx.alloc(d.n * d.ob) for _ in range(copies)]
            ctx.grouped([{"w": d.w, "out": o, "scales": d.s, "rows": 4096, "cols": 4096, "fmt": case["fmt"],
                          "scale_mode": case["scale_mode"], "loras": d.loras} for o in outs])
            got = []
            for o in outs:
                g = np.empty((4096, 4096), np.uint16)
                ctx.download(o, g)
                got.append(g)
        ctx.dequant(d.w, 4096, 4096, case["fmt"], case["scale_mode"], d.s, d.out)
        deq = d.result()
        for g in got:
            assert np.array_equal(g, deq)
    finally:
        for o in outs:
            ctx.free(o)
        d.free()


@pytest.mark.parametrize("ranks", [((64, 1.0),), ((32, 1.0), (128, 0.5))])
def test_row_and_column_permutation_equivariance(ctx, ranks):
    """Rows and columns are independent and every element's sum runs in the
    same order wherever it sits, so permuting the rows of W, the scales and B
    (or the columns of W and A) permutes the output the same way, bit for bit,
    at the full 4096 x 4104 size (a partial column band included). Catches a
    factor row or column paired with the wrong output."""
    log("case: permutation", ranks)
    rows, cols = 4096, 4104
    case = synth.tensor_case(4545, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=ranks)
    rng = np.random.default_rng(45)
    p, q = rng.permutation(rows), rng.permutation(cols)
    base = run_case(ctx, case)
    by_rows = dict(case, w=np.ascontiguousarray(case["w"][p]), scales=np.ascontiguousarray(case["scales"][p]),
                   loras=[(np.ascontiguousarray(b[p]), a, r, c) for (b, a, r, c) in case["loras"]])
    assert np.array_equal(run_case(ctx, by_rows), base[p])
    by_cols = dict(case, w=np.ascontiguousarray(case["w"][:, q]),
                   loras=[(b, np.ascontiguousarray(a[:, q]), r, c) for (b, a, r, c) in case["loras"]])
    assert np.array_equal(run_case(ctx, by_cols), base[:, q])


def test_fused_f32_output(ctx):
    """f32 output (the reference's own HostTensor type): within the f32
    forward-error bound of both orders, 2*(rank+4)*2^-24*(|deq|+sum|cBA|)."""
    log("case: fused f32 out")
    case = synth.tensor_case(55, 512, 1024, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
    got = run_case(ctx, case, lw.OUT_F32).astype(np.float64)
    ref = U.oracle_f32(case).astype(np.float64)
    w, f, m, s, loras = U.oracle_args(case)
    import oracle_lib as O
    bound = O.abs_bound_rows(w, f, m, s, loras)
    assert np.all(np.abs(got - ref) <= 2 * (64 + 4) * 2.0 ** -24 * bound)


@pytest.mark.parametrize("rows,cols,ranks", [(9, 13, ((2, 0.75),)), (40, 100, ((3, 1.0), (5, 0.5))), (16, 24, ((4, 1.5),))])
def test_generic_path_bit_exact(ctx, rows, cols, ranks):
    """Ranks or widths the tiled kernel does not take run in the reference's
    own operation order, so the result is bit-identical to the oracle."""
    log("case: generic", rows, cols, ranks)
    case = synth.tensor_case(rows + cols, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=ranks)
    for out_dtype in (lw.OUT_BF16, lw.OUT_F32):
        got = run_case(ctx, case, out_dtype)
        ref = U.oracle_bf16(case) if out_dtype == lw.OUT_BF16 else U.oracle_f32(case)
        assert np.array_equal(got.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32),
                              ref.view(np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32))


def test_fused_nan_inf_codes(ctx):
    """NaN and Inf codes through the fused path: NaN stays the reference's
    f32::NAN (bf16 0x7FC0), +-Inf plus a finite delta stays +-Inf."""
    log("case: fused nan/inf")
    rng = np.random.default_rng(5)
    b, a = synth.lora_factors(rng, 64, 256, 16)
    case = all_codes_case(lw.FMT_E5M2, lw.SCALE_ROW, loras=[(b, a, 16, 1.0)])
    got = run_case(ctx, case)
    U.compare_lora_bf16(case, got)


def test_many_grouped_calls_in_flight(ctx):
    """48 grouped calls queued without a wait, each with its own outputs: the
    host runs ahead of the GPU through the ring of job-table slots, so every
    slot's host copy and device table is reused while earlier calls are still
    queued. Every output must equal the tensor's own single-call result, and
    an empty grouped call is a no-op."""
    log("case: grouped calls in flight")
    cases = [synth.tensor_case(4800 + k, 4096, 4096, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
             for k in range(2)]
    devs = [U.Dev(ctx, c) for c in cases]
    outs = []
    try:
        singles = []
        for d in devs:
            d.run()
            singles.append(d.result())
        n_calls = 48
        outs = [[ctx.alloc(d.n * d.ob) for d in devs] for _ in range(n_calls)]
        for call in outs:
            for o, d in zip(call, devs):
                ctx.memset(o, 0xFF, d.n * d.ob)
        ctx.synchronize()
        descs = [lw.Context.make_descs([{"w": d.w, "out": o, "scales": d.s, "rows": d.case["rows"],
                                         "cols": d.case["cols"], "fmt": d.case["fmt"],
                                         "scale_mode": d.case["scale_mode"], "loras": d.loras}
                                        for o, d in zip(call, devs)]) for call in outs]
        for arr in descs:
            ctx.grouped(arr)
        ctx.grouped([])
        ctx.synchronize()
        for k, call in enumerate(outs):
            for o, d, s in zip(call, devs, singles):
                got = np.empty_like(s)
                ctx.download(o, got)
                assert np.array_equal(got, s), "call %d" % k
    finally:
        for call in outs:
            for o in call:
                ctx.free(o)
        for d in devs:
            d.free()


def test_grouped_calls_with_device_job_tables(ctx):
    """Grouped launches whose job records do not fit the kernel arguments
    (30 single-LoRA jobs; 14 jobs with two LoRAs, 5 K-steps) read them from
    the device table ring: 24 calls queued without a wait reuse every slot.
    Every output must equal the tensor's own single-call result."""
    log("case: grouped calls with device job tables")
    cases = [synth.tensor_case(5000 + k, 256, 256, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
             for k in range(30)]
    cases += [synth.tensor_case(5100 + k, 130, 264, synth.E5M2, synth.SCALE_TENSOR, loras=((32, 1.0), (128, 0.5)))
              for k in range(14)]
    devs = [U.Dev(ctx, c) for c in cases]
    outs = []
    try:
        singles = []
        for d in devs:
            d.run()
            singles.append(d.result())
        n_calls = 24
        outs = [[ctx.alloc(d.n * d.ob) for d in devs] for _ in range(n_calls)]
        for call in outs:
            for o, d in zip(call, devs):
                ctx.memset(o, 0xFF, d.n * d.ob)
        ctx.synchronize()
        for call in outs:
            ctx.grouped([{"w": d.w, "out": o, "scales": d.s, "rows": d.case["rows"], "cols": d.case["cols"],
                          "fmt": d.case["fmt"], "scale_mode": d.case["scale_mode"], "loras": d.loras}
                         for o, d in zip(call, devs)])
        ctx.synchronize()
        for k, call in enumerate(outs):
            for o, d, s in zip(call, devs, singles):
                got = np.empty_like(s)
                ctx.download(o, got)
                assert np.array_equal(got, s), "call %d" % k
    finally:
        for call in outs:
            for o in call:
                ctx.free(o)
        for d in devs:
            d.free()


@pytest.mark.parametrize("loras", [((64, 1.0),), ((32, 1.0), (32, -0.5))], ids=["r64", "r32+r32"])
def test_grouped_call_inline_records_beyond_first_workgroup_array(ctx, loras):
    """20 tensors of 2 K-steps in one grouped call: their records (20 x 128
    bytes) still travel in the kernel arguments, but there are more of them
    than the 16-entry array of first workgroups holds, so a workgroup finds
    its record by a binary search over the inline records (the case of two
    DiT blocks in one call). Every output equals the tensor's own
    single-call result."""
    log("case: 20 inline records", loras)
    shapes = [(64 + 24 * k, 128 + 8 * (k % 7) * 8) for k in range(20)]
    cases = [synth.tensor_case(5200 + k, r, c, synth.E4M3FN if k % 2 else synth.E5M2,
                               synth.SCALE_ROW if k % 3 else synth.SCALE_TENSOR, loras=loras)
             for k, (r, c) in enumerate(shapes)]
    devs = [U.Dev(ctx, c) for c in cases]
    try:
        singles = []
        for d in devs:
            d.run()
            singles.append(d.result())
        for d in devs:
            ctx.memset(d.out, 0xFF, d.n * d.ob)
        ctx.grouped([{"w": d.w, "out": d.out, "scales": d.s, "rows": d.case["rows"], "cols": d.case["cols"],
                      "fmt": d.case["fmt"], "scale_mode": d.case["scale_mode"], "loras": d.loras} for d in devs])
        for k, (d, s) in enumerate(zip(devs, singles)):
            assert np.array_equal(d.result(), s), "tensor %d" % k
    finally:
        for d in devs:
            d.free()


def test_grouped_block_matches_single_calls(ctx):
    """A grouped launch over mixed tensors equals per-tensor calls bit for bit."""
    log("case: grouped vs single")
    cases = [
        synth.tensor_case(11, 256, 512, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),)),
        synth.tensor_case(12, 384, 256, synth.E5M2, synth.SCALE_TENSOR, loras=((32, 1.0), (16, 0.5))),
        synth.tensor_case(13, 100, 72, synth.E4M3FN, synth.SCALE_ROW, loras=((8, 1.0),)),
        synth.tensor_case(14, 64, 64, synth.E4M3FN, synth.SCALE_NONE, loras=()),
        synth.tensor_case(15, 33, 21, synth.E4M3FN, synth.SCALE_ROW, loras=((2, 0.5),)),
    ]
    devs = [U.Dev(ctx, c) for c in cases]
    try:
        singles = []
        for d in devs:
            d.run()
            singles.append(d.result())
        for d in devs:
            ctx.memset(d.out, 0xFF, d.n * d.ob)
        ctx.grouped([{"w": d.w, "out": d.out, "scales": d.s, "rows": d.case["rows"], "cols": d.case["cols"],
                      "fmt": d.case["fmt"], "scale_mode": d.case["scale_mode"], "loras": d.loras} for d in devs])
        for d, s in zip(devs, singles):
            assert np.array_equal(d.result(), s)
    finally:
        for d in devs:
            d.free()


def test_dit_block_sampled_rows(ctx):
    """One DiT block (8 x 4096^2, 16384 x 4096, 4096 x 16384), per-row scales,
    rank-64 LoRA on every tensor, materialised in one grouped call; each tensor
    checked against the oracle on 96 sampled rows plus the first and last."""
    log("case: DiT block")
    rng = np.random.default_rng(0)
    cases, devs = [], []
    try:
        for k, (name, rows, cols) in enumerate(synth.BLOCK_LINEARS):
            c = synth.tensor_case(3000 + k, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
            cases.append(c)
            devs.append(U.Dev(ctx, c))
        ctx.grouped([{"w": d.w, "out": d.out, "scales": d.s, "rows": d.case["rows"], "cols": d.case["cols"],
                      "fmt": d.case["fmt"], "scale_mode": d.case["scale_mode"], "loras": d.loras} for d in devs])
        for d, c in zip(devs, cases):
            got = d.result()
            sel = np.unique(np.concatenate([[0, c["rows"] - 1], rng.choice(c["rows"], 96, replace=False)]))
            U.compare_lora_bf16(c, got[sel], row_sel=sel)
    finally:
        for d in devs:
            d.free()


def test_mixed_format_block_sampled_rows(ctx):
    """The mixed-format DiT block at full size in one grouped call: attention
    e4m3fn with one scale, FFN e5m2 with row scales, the 4096 x 4104 and
    4104 x 16384 edge tensors, and two stacked LoRAs (rank 32, coefficient 1;
    rank 128, coefficient 0.5) on every tensor; 48 sampled rows plus the first
    and last of each tensor against the oracle."""
    log("case: mixed-format block")
    rng = np.random.default_rng(5)
    shapes = [(nm, r, c, nm.startswith("ff.")) for nm, r, c in synth.BLOCK_LINEARS]
    shapes += [("edge.proj_a", 4096, 4104, False), ("edge.proj_b", 4104, 16384, True)]
    cases, devs = [], []
    try:
        for k, (name, rows, cols, ffn) in enumerate(shapes):
            fmt, sm = (synth.E5M2, synth.SCALE_ROW) if ffn else (synth.E4M3FN, synth.SCALE_TENSOR)
            c = synth.tensor_case(5000 + k, rows, cols, fmt, sm, loras=((32, 1.0), (128, 0.5)))
            cases.append(c)
            devs.append(U.Dev(ctx, c))
        ctx.grouped([{"w": d.w, "out": d.out, "scales": d.s, "rows": d.case["rows"], "cols": d.case["cols"],
                      "fmt": d.case["fmt"], "scale_mode": d.case["scale_mode"], "loras": d.loras} for d in devs])
        for d, c in zip(devs, cases):
            got = d.result()
            sel = np.unique(np.concatenate([[0, c["rows"] - 1], rng.choice(c["rows"], 48, replace=False)]))
            U.compare_lora_bf16(c, got[sel], row_sel=sel)
    finally:
        for d in devs:
            d.free()


def test_invalid_arguments_report_status(ctx):
    log("case: errors")
    p = ctx.alloc(1024)
    try:
        with pytest.raises(lw.InvalidArgument):
            ctx.dequant(p, -1, 4, lw.FMT_E4M3FN, lw.SCALE_NONE, None, p)
        with pytest.raises(lw.UnsupportedDtype):
            ctx.dequant(p, 4, 4, 7, lw.SCALE_NONE, None, p)
        with pytest.raises(lw.InvalidArgument):
            ctx.dequant(p, 4, 4, lw.FMT_E4M3FN, lw.SCALE_ROW, None, p)
        with pytest.raises(lw.InvalidArgument):
            ctx.dequant(None, 4, 4, lw.FMT_E4M3FN, lw.SCALE_NONE, None, p)
        with pytest.raises(lw.LoraRankMismatch):
            ctx.dequant_lora(p, 4, 4, lw.FMT_E4M3FN, lw.SCALE_NONE, None, [(p, p, 0, 1.0)], p)
        with pytest.raises(lw.InvalidArgument):
            ctx.dequant_lora(p, 4, 4, lw.FMT_E4M3FN, lw.SCALE_NONE, None, [(p, p, 1, 1.0)] * 5, p)
        with pytest.raises(lw.InvalidArgument):
            ctx.dequant(p, 1 << 40, 1 << 40, lw.FMT_E4M3FN, lw.SCALE_NONE, None, p)
        with pytest.raises(lw.OutOfMemory):
            ctx.alloc(1 << 50)
        ctx.dequant(p, 0, 4, lw.FMT_E4M3FN, lw.SCALE_NONE, None, p)  # empty: no-op
        ctx.synchronize()
    finally:
        ctx.free(p)


def test_undersized_buffers_rejected_before_launch(ctx):
    """A buffer smaller than the tensor it is passed for is an InvalidArgument
    (checked on the host against the allocation's extent), never a launch."""
    log("case: undersized buffers")
    small, big = ctx.alloc(1024), ctx.alloc(1 << 20)
    try:
        E4, NONE, ROW = lw.FMT_E4M3FN, lw.SCALE_NONE, lw.SCALE_ROW
        with pytest.raises(lw.InvalidArgument, match="weight"):
            ctx.dequant(small, 64, 64, E4, NONE, None, big)
        with pytest.raises(lw.InvalidArgument, match="output"):
            ctx.dequant(big, 64, 64, E4, NONE, None, small)
        with pytest.raises(lw.InvalidArgument, match="scales"):
            ctx.dequant(big, 512, 64, E4, ROW, small, big)
        with pytest.raises(lw.InvalidArgument, match="LoRA B"):
            ctx.dequant_lora(big, 64, 64, E4, NONE, None, [(small, big, 64, 1.0)], big)
        with pytest.raises(lw.InvalidArgument, match="LoRA A"):
            ctx.dequant_lora(big, 64, 64, E4, NONE, None, [(big, small, 64, 1.0)], big)
        with pytest.raises(lw.InvalidArgument, match="weight"):
            ctx.dequant(big + (1 << 20) - 100, 1, 200, E4, NONE, None, big)
        with pytest.raises(lw.InvalidArgument, match="upload destination"):
            ctx.upload(np.zeros(1 << 16, np.uint8), small)
        with pytest.raises(lw.InvalidArgument, match="download source"):
            ctx.download(small, np.empty(1 << 16, np.uint8))
        with pytest.raises(lw.InvalidArgument, match="memset destination"):
            ctx.memset(small, 0, 1 << 16)
        ctx.synchronize()
    finally:
        ctx.free(small)
        ctx.free(big)


def test_tensor_beyond_32bit_byte_offsets(ctx):
    """A 16392 x 65536 e5m2 tensor (2^30 + 2^19 elements, every byte value,
    NaN codes included) with per-row scales and f32 output: 4 GiB of output,
    byte offsets past 2^32. Without a LoRA it takes the linear dequant kernel
    (above the tiled kernel's 2^27 elements); with a rank-16 LoRA the
    reference-order kernel (past the fused kernels' 32-bit offsets). The first,
    second and last rows and 30 sampled ones match the oracle bit for bit."""
    log("case: 16392 x 65536 e5m2, f32 out")
    rows, cols = 16392, 65536
    rng = np.random.default_rng(9090)
    w = rng.integers(0, 256, size=(rows, cols), dtype=np.uint8)
    b, a = synth.lora_factors(rng, rows, cols, 16)
    case = {"w": w, "scales": synth.scales(rng, rows, synth.SCALE_ROW), "loras": [], "rows": rows, "cols": cols,
            "fmt": synth.E5M2, "scale_mode": synth.SCALE_ROW}
    sel = np.unique(np.concatenate([[0, 1, rows - 1], rng.choice(rows, 30, replace=False)]))
    d = U.Dev(ctx, case, lw.OUT_F32)
    try:
        for loras in ([], [(b, a, 16, 0.75)]):
            case["loras"] = loras
            d.loras = [(d._put(lb), d._put(la), r, c, lw.FACTOR_BF16) for (lb, la, r, c) in loras]
            d.run()
            got = np.empty((len(sel), cols), np.float32)
            for k, r in enumerate(sel):
                ctx.download(d.out + int(r) * cols * 4, got[k])
            ref = U.oracle_f32(case, row_sel=sel)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), "n_loras %d" % len(loras)
    finally:
        d.free()


def test_upload_download_round_trip(ctx):
    log("case: round trip")
    rng = np.random.default_rng(1)
    x = rng.integers(0, 256, size=(3 << 20) + 7, dtype=np.uint8)
    p = ctx.alloc(x.nbytes)
    try:
        ctx.upload(x, p)
        y = np.empty_like(x)
        ctx.download(p, y)
        assert np.array_equal(x, y)
    finally:
        ctx.free(p)


def test_upload_is_ordered_after_queued_work(ctx):
    """ltxw_upload runs in call order: refilling a device buffer while a
    kernel that reads it is still queued, or right after a queued memset of
    it, gives every operation the data it was queued with."""
    log("case: upload ordering")
    rng = np.random.default_rng(12)
    rows, cols = 2048, 4096
    cases = [synth.tensor_case(1200 + k, rows, cols, synth.E4M3FN, synth.SCALE_TENSOR, loras=()) for k in range(3)]
    x = ctx.alloc(rows * cols)
    sc = ctx.alloc(4 * 3)
    outs = [ctx.alloc(rows * cols * 2) for _ in cases]
    try:
        for k, c in enumerate(cases):
            ctx.upload(c["scales"], sc + 4 * k)
        # Queue: several big kernels ahead, then dequant(x) -> out0, refill x,
        # dequant(x) -> out1, memset x, refill x, dequant(x) -> out2.
        busy = ctx.alloc(rows * cols * 2)
        for _ in range(8):
            ctx.dequant(x, rows, cols, lw.FMT_E4M3FN, lw.SCALE_TENSOR, sc, busy)
        ctx.upload(cases[0]["w"], x)
        ctx.dequant(x, rows, cols, lw.FMT_E4M3FN, lw.SCALE_TENSOR, sc, outs[0])
        ctx.upload(cases[1]["w"], x)
        ctx.dequant(x, rows, cols, lw.FMT_E4M3FN, lw.SCALE_TENSOR, sc + 4, outs[1])
        ctx.memset(x, 0, rows * cols)
        ctx.upload(cases[2]["w"], x)
        ctx.dequant(x, rows, cols, lw.FMT_E4M3FN, lw.SCALE_TENSOR, sc + 8, outs[2])
        ctx.synchronize()
        ctx.free(busy)
        for c, o in zip(cases, outs):
            got = np.empty((rows, cols), np.uint16)
            ctx.download(o, got)
            assert np.array_equal(got, U.oracle_bf16(c))
    finally:
        for p in [x, sc] + outs:
            ctx.free(p)
    del rng


# ---------------------------------------------------------------------------
# Exact mode (LTXW_DESC_EXACT): the reference's own operation order, bit for bit
# ---------------------------------------------------------------------------
def run_grouped(ctx, cases, out_dtype=lw.OUT_BF16, flags=0):
    devs = [U.Dev(ctx, c, out_dtype) for c in cases]
    try:
        descs = [{"w": d.w, "out": d.out, "scales": d.s, "rows": c["rows"], "cols": c["cols"], "fmt": c["fmt"],
                  "scale_mode": c["scale_mode"], "out_dtype": out_dtype, "loras": d.loras, "flags": flags}
                 for d, c in zip(devs, cases)]
        ctx.grouped(descs)
        return [d.result() for d in devs]
    finally:
        for d in devs:
            d.free()


@pytest.mark.parametrize("rows,cols,ranks,fmt,scale_mode", [
    (512, 1024, ((64, 1.0),), synth.E4M3FN, synth.SCALE_ROW),
    (300, 520, ((32, 1.0), (128, 0.5)), synth.E5M2, synth.SCALE_ROW),
    (129, 136, ((8, 0.75),), synth.E4M3FN, synth.SCALE_TENSOR),
    (64, 8, ((3, 1.25), (5, -0.5), (2, 2.0)), synth.E5M2, synth.SCALE_NONE),
])
def test_exact_mode_bit_exact(ctx, rows, cols, ranks, fmt, scale_mode):
    """With LTXW_DESC_EXACT every delta runs in the reference's order: bf16 and
    f32 outputs equal the oracle bit for bit, shapes the MFMA path would take
    included."""
    log("case: exact", rows, cols, ranks, fmt, scale_mode)
    case = synth.tensor_case(rows * 7 + cols, rows, cols, fmt, scale_mode, loras=ranks)
    for out_dtype in (lw.OUT_BF16, lw.OUT_F32):
        got, = run_grouped(ctx, [case], out_dtype, flags=lw.DESC_EXACT)
        ref = U.oracle_bf16(case) if out_dtype == lw.OUT_BF16 else U.oracle_f32(case)
        view = np.uint16 if out_dtype == lw.OUT_BF16 else np.uint32
        assert np.array_equal(got.view(view), ref.view(view))


def test_exact_mode_nan_inf_codes(ctx):
    log("case: exact nan/inf")
    for fmt in (lw.FMT_E4M3FN, lw.FMT_E5M2):
        case = all_codes_case(fmt, lw.SCALE_ROW, rows=64, cols=256)
        rng = np.random.default_rng(5)
        b, a = synth.lora_factors(rng, 64, 256, 32)
        case["loras"] = [(b, a, 32, 1.0)]
        got, = run_grouped(ctx, [case], lw.OUT_BF16, flags=lw.DESC_EXACT)
        assert np.array_equal(got, U.oracle_bf16(case))


def test_exact_and_fused_agree_within_tolerance(ctx):
    """The MFMA path stays within the stated tolerance of the exact path's
    (= the reference's) result on the same launch."""
    log("case: exact vs fused")
    case = synth.tensor_case(991, 512, 512, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
    exact, = run_grouped(ctx, [case], flags=lw.DESC_EXACT)
    fused, = run_grouped(ctx, [case], flags=0)
    assert np.array_equal(exact, U.oracle_bf16(case))
    assert int(np.abs(U.bf16_ordered(exact) - U.bf16_ordered(fused)).max()) <= 1
