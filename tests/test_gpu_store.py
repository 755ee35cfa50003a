"""GPU tests of the weight store: `read` and `materialize` through
include/ltxw_store.h against the oracle and the reference's own expected
values (crates/ltx-weights/tests/integration.rs).

Bars: dequant (no LoRA) and every path that runs in the reference's
operation order (non-bf16 factors, non-FP8 bases) bit-exact in f32 and bf16;
bf16 factors on FP8 bases (MFMA path) within 1 bf16 ulp + the Frobenius
bound of gpu_util.compare_lora_bf16.
"""
import ctypes

import numpy as np
import pytest

import gpu_util as U
import ltx_weights as lw
import oracle_lib as O
import st_io
from ltx_weights import synth
from ltx_weights.store import MAT_EXACT, MAT_MFMA, MAT_ROW_SCALES, MAT_SCALE_FIRST, KeyMap, LoraFile, WeightStore

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def ctx():
    log("test_gpu_store: context on device 0")
    c = lw.Context(0)
    yield c
    c.close()


@pytest.fixture
def tmp(tmp_path):
    class W:
        n = 0

        def __call__(self, tensors, metadata=None):
            W.n += 1
            p = tmp_path / f"g{W.n}.safetensors"
            st_io.write(p, tensors, metadata)
            return p

    return W()


def f32(*v):
    return np.array(v, dtype=np.float32)


def bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------------------
# The reference's integration tests, through the device read path
# ---------------------------------------------------------------------------
def test_identity_reads_f32_f16_bf16(ctx, tmp):
    log("identity reads")
    vals = f32(0.5, 1.0, -1.0, 2.0)
    bf = synth.bf16_from_f64([3.14, -2.71, 0.0, 1.0])
    p = tmp([("f", "F32", [2, 2], f32(1, 2, 3, 4)), ("h", "F16", [4], vals.astype(np.float16).view(np.uint16)),
             ("b", "BF16", [4], bf)])
    s = WeightStore.open([p])
    assert s.read("f", ctx)[1].tolist() == [[1, 2], [3, 4]]
    assert np.array_equal(s.read("h", ctx)[1], vals)
    assert np.array_equal(bits(s.read("b", ctx)[1]), bits(O.decode(bf, O.BF16)))


def test_fp8_with_and_without_scale(ctx, tmp):
    log("fp8 scale")
    p = tmp([("w", "F8_E4M3", [1], np.array([0x38], np.uint8)), ("v", "F8_E4M3", [1], np.array([0x38], np.uint8)),
             ("v_scale", "F32", [1], f32(3.0))])
    s = WeightStore.open([p])
    assert s.read("w", ctx)[1].tolist() == [1.0]
    assert s.read("v", ctx)[1].tolist() == [3.0]


def test_non_fp8_scale_sibling_not_applied(ctx, tmp):
    p = tmp([("w", "F32", [1], f32(2.0)), ("w_scale", "F32", [1], f32(100.0))])
    s = WeightStore.open([p])
    assert s.read("w", ctx)[1].tolist() == [2.0]
    assert s.read("w_scale", ctx)[1].tolist() == [100.0]


def test_lora_merge_basic_alpha_and_stacking_values(ctx, tmp):
    log("lora merge values")
    base = tmp([("layer.weight", "F32", [2, 2], f32(1, 0, 0, 1)), ("w.weight", "F32", [2, 2], f32(0, 0, 0, 0)),
                ("s.weight", "F32", [2, 2], f32(1, 0, 0, 1))])
    store = WeightStore.open([base])
    store.merge_lora(LoraFile.open(tmp([("layer.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                                        ("layer.lora_B.weight", "F32", [2, 1], f32(3, 4)),
                                        ("w.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                                        ("w.lora_B.weight", "F32", [2, 1], f32(3, 4)),
                                        ("w.alpha", "F32", [1], f32(2.0)),
                                        ("s.lora_A.weight", "F32", [1, 2], f32(1, 2)),
                                        ("s.lora_B.weight", "F32", [2, 1], f32(3, 4))])), 1.0)
    store.merge_lora(LoraFile.open(tmp([("s.lora_A.weight", "F32", [2, 2], f32(1, 0, 0, 1)),
                                        ("s.lora_B.weight", "F32", [2, 2], f32(2, 0, 0, -2))])), 0.5)
    assert store.read("layer.weight", ctx)[1].tolist() == [[4, 6], [4, 9]]
    assert store.read("w.weight", ctx)[1].tolist() == [[6, 12], [8, 16]]
    assert store.read("s.weight", ctx)[1].tolist() == [[5, 6], [4, 8]]


def _fixture_file(tmp, stem):
    """A reference fixture (crates/ltx-weights/tests/fixtures/<stem>.safetensors)
    rewritten from the committed vectors, with its metadata."""
    import json

    import golden_checks as G

    with open(G.REF_FIXTURES) as f:
        meta = json.load(f)["files"][stem]["metadata"]
    ts = [(name, dt, shape, arr) for name, (dt, shape, arr) in G.load_fixture_tensors(stem).items()]
    return tmp(ts, meta or None)


def test_reference_parity_fixture_lora_merge_bf16(ctx, tmp):
    """crates/ltx-weights/tests/parity.rs:23-47 through the device path: bf16
    base, f32 rank-2 factors with alpha 4, strength 0.75. The reference
    allows 5e-2; here `read` must equal the oracle's f32 bit for bit and its
    bf16 rounding (read, and materialize in both orders) must equal the
    fixture's expected bf16 tensor, 32/32."""
    log("reference fixture: lora parity")
    store = WeightStore.open([_fixture_file(tmp, "lora_parity_base")])
    report = store.merge_lora(LoraFile.open(_fixture_file(tmp, "lora_parity_lora")), 0.75)
    assert "layer.weight" in report.matched_keys
    got = store.read("layer.weight", ctx)[1]
    expected_store = WeightStore.open([_fixture_file(tmp, "lora_parity_expected")])
    expected = expected_store.read("layer.weight", ctx)[1]
    assert got.shape == expected.shape == (8, 4)
    assert np.all(np.abs(got - expected) <= 5e-2)  # the reference's own bar
    import golden_checks as G

    base, a, b, alpha, exp_bits = G.lora_fixture_inputs()
    want = O.read_f32(base, O.BF16, loras=[(b, a, O.F32, O.lora_coeff(0.75, alpha, 2))])
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(O.read_bf16(got, O.F32), exp_bits)
    for flags in (0, MAT_EXACT):
        t = store.materialize_bf16(ctx, ["layer.weight"], flags=flags)["layer.weight"]
        try:
            assert np.array_equal(t.to_numpy(), exp_bits), flags
        finally:
            t.free()


def test_reference_parity_fixture_fp8_e4m3fn_with_scale(ctx, tmp):
    """crates/ltx-weights/tests/parity.rs:51-75 through the device path:
    4x4 e4m3fn with a scalar scale; 16/16 f32 bit-identical to the fixture's
    expected tensor (the reference allows 1e-5)."""
    log("reference fixture: fp8 parity")
    store = WeightStore.open([_fixture_file(tmp, "fp8_e4m3fn_parity")])
    got = store.read("w", ctx)[1]
    expected = WeightStore.open([_fixture_file(tmp, "fp8_e4m3fn_expected")]).read("w", ctx)[1]
    assert got.shape == expected.shape == (4, 4)
    assert np.array_equal(bits(got), bits(expected))
    t = store.materialize_bf16(ctx, ["w"])["w"]
    try:
        assert np.array_equal(t.to_numpy(), O.read_bf16(expected, O.F32))
    finally:
        t.free()


def test_read_errors(ctx, tmp):
    p = tmp([("w", "I32", [2], np.array([42, -1], np.int32)), ("x", "F32", [1], f32(0))])
    s = WeightStore.open([p])
    with pytest.raises(lw.UnsupportedDtype):
        s.read("w", ctx)
    with pytest.raises(lw.MissingKey):
        s.read("does_not_exist", ctx)


# ---------------------------------------------------------------------------
# Random cases against the oracle
# ---------------------------------------------------------------------------
FACTOR_DT = {"F32": O.F32, "F16": O.F16, "BF16": O.BF16, "F8_E4M3": O.E4M3FN, "F8_E5M2": O.E5M2}


def factor_bits(rng, dt, shape, std):
    x = rng.normal(0.0, std, size=shape)
    if dt == "F32":
        return x.astype(np.float32)
    if dt == "F16":
        return x.astype(np.float16).view(np.uint16)
    if dt == "BF16":
        return synth.bf16_from_f64(x)
    codes = synth.E4M3FN_CODES if dt == "F8_E4M3" else synth.E5M2_FINITE_CODES
    return codes[rng.integers(0, len(codes), size=shape)]


def base_bits(rng, dt, shape):
    if dt in ("F8_E4M3", "F8_E5M2"):
        codes = synth.E4M3FN_CODES if dt == "F8_E4M3" else synth.E5M2_FINITE_CODES
        return codes[rng.integers(0, len(codes), size=shape)]
    return factor_bits(rng, dt, shape, 1.0)


@pytest.mark.parametrize("base_dt,factor_dt,ranks,shape,scale", [
    ("F8_E4M3", "F32", [3], (24, 40), "row"),
    ("F8_E5M2", "F16", [5, 2], (33, 17), "tensor"),
    ("F8_E4M3", "F8_E4M3", [4], (16, 16), "row"),
    ("BF16", "BF16", [8], (20, 64), None),
    ("F16", "F32", [2], (9, 31), None),
    ("F32", "BF16", [16, 8], (12, 48), None),
    ("F8_E4M3", "BF16", [6], (10, 30), "tensor"),   # cols % 8 != 0: generic path
])
def test_reference_order_paths_bit_exact(ctx, tmp, base_dt, factor_dt, ranks, shape, scale):
    """Every path that keeps the reference's operation order matches the
    oracle's f32 bit for bit (and its bf16 rounding): the tensors the MFMA
    kernels do not take, and, with MAT_EXACT, those they do (here the bf16
    base with bf16 factors)."""
    log("reference-order case", base_dt, factor_dt, ranks, shape, scale)
    rng = np.random.default_rng(hash((base_dt, factor_dt, tuple(ranks), shape)) % (1 << 31))
    rows, cols = shape
    w = base_bits(rng, base_dt, (rows, cols))
    ts = [("t.weight", base_dt, [rows, cols], w)]
    sc = None
    if scale == "row":
        sc = rng.uniform(1e-3, 1e-1, rows).astype(np.float32)
        ts.append(("t.weight_scale", "F32", [rows], sc))
    elif scale == "tensor":
        sc = rng.uniform(1e-3, 1e-1, 1).astype(np.float32)
        ts.append(("t.weight_scale", "F32", [], sc))
    store = WeightStore.open([tmp(ts)])
    loras = []
    for k, r in enumerate(ranks):
        a = factor_bits(rng, factor_dt, (r, cols), 0.05)
        b = factor_bits(rng, factor_dt, (rows, r), 0.05)
        strength = [1.0, 0.5, 0.25][k]
        store.merge_lora(LoraFile.open(tmp([("t.lora_A.weight", factor_dt, [r, cols], a),
                                            ("t.lora_B.weight", factor_dt, [rows, r], b)])), strength)
        loras.append((b.reshape(rows, r), a.reshape(r, cols), FACTOR_DT[factor_dt], O.lora_coeff(strength, None, r)))
    smode = {None: O.SCALE_NONE, "row": O.SCALE_ROW, "tensor": O.SCALE_TENSOR}[scale]
    want = O.read_f32(w.reshape(rows, cols), O.DTYPE_CODES[base_dt], smode, sc, loras)
    got = store.read("t.weight", ctx, flags=MAT_ROW_SCALES)[1]  # reference order is read's default
    assert np.array_equal(bits(got), bits(want))
    # bf16 materialisation of the same key = RNE of that f32.
    out = store.materialize_bf16(ctx, ["t.weight"], flags=MAT_EXACT)["t.weight"]
    try:
        assert np.array_equal(out.to_numpy(), O.read_bf16(w.reshape(rows, cols), O.DTYPE_CODES[base_dt], smode, sc,
                                                          loras))
    finally:
        out.free()


def test_fused_path_through_store(ctx, tmp):
    log("fused through store")
    rng = np.random.default_rng(11)
    case = synth.tensor_case(11, 256, 512, synth.E5M2, synth.SCALE_ROW, loras=((64, 1.0), (32, 0.5)))
    ts = [("m.weight", "F8_E5M2", [256, 512], case["w"]), ("m.weight_scale", "F32", [256], case["scales"])]
    store = WeightStore.open([tmp(ts)])
    for k, (b, a, r, c) in enumerate(case["loras"]):
        store.merge_lora(LoraFile.open(tmp([("m.lora_A.weight", "BF16", [r, 512], a),
                                            ("m.lora_B.weight", "BF16", [256, r], b)])), c)
    out = store.materialize_bf16(ctx, ["m.weight"], flags=MAT_MFMA)["m.weight"]
    try:
        stats = U.compare_lora_bf16(case, out.to_numpy())
    finally:
        out.free()
    log("fused via store:", stats)
    # Without MAT_MFMA: the reference's operation order, bit for bit.
    out = store.materialize_bf16(ctx, ["m.weight"])["m.weight"]
    try:
        assert np.array_equal(out.to_numpy(), U.oracle_bf16(case))
    finally:
        out.free()
    del rng


def test_scale_policy_and_dtypes(ctx, tmp):
    """`read` follows the reference's rule: every scale tensor scales by its
    element 0 (store.rs:498-508, :732-735), also one of shape[0] elements;
    MAT_ROW_SCALES (and materialize by default) scales row o by element o.
    Scales in bf16/f16 widen exactly."""
    log("scale policy")
    rng = np.random.default_rng(4)
    rows, cols = 16, 64
    w = synth.E4M3FN_CODES[rng.integers(0, 254, (rows, cols))]
    s16 = synth.bf16_from_f64(rng.uniform(1e-3, 1e-1, rows))
    store = WeightStore.open([tmp([("w", "F8_E4M3", [rows, cols], w), ("w_scale", "BF16", [rows], s16)])])
    sc = O.decode(s16, O.BF16)
    want_first = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, sc[:1])
    want_row = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, sc)
    assert np.array_equal(bits(store.read("w", ctx)[1]), bits(want_first))
    assert np.array_equal(bits(store.read("w", ctx, flags=MAT_SCALE_FIRST)[1]), bits(want_first))
    assert np.array_equal(bits(store.read("w", ctx, flags=MAT_ROW_SCALES)[1]), bits(want_row))
    for flags, want in ((0, want_row), (MAT_SCALE_FIRST, want_first)):
        out = ctx.alloc(rows * cols * 4)
        try:
            store.materialize(ctx, ["w"], [out], lw.OUT_F32, flags)
            got = np.empty((rows, cols), np.float32)
            ctx.download(out, got)
            assert np.array_equal(bits(got), bits(want)), flags
        finally:
            ctx.free(out)
    with pytest.raises(lw.InvalidArgument):
        store.read("w", ctx, flags=MAT_SCALE_FIRST | MAT_ROW_SCALES)
    with pytest.raises(lw.InvalidArgument):
        store.read("w", ctx, flags=MAT_EXACT | MAT_MFMA)
    # A scale of another length scales by element 0 (store.rs:732-735).
    store2 = WeightStore.open([tmp([("w", "F8_E4M3", [rows, cols], w),
                                    ("w_scale", "F16", [3], np.array([0.5, 2, 4], np.float16).view(np.uint16))])])
    assert np.array_equal(bits(store2.read("w", ctx)[1]), bits(O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, f32(0.5))))
    # An empty scale tensor scales by 1.0 (and so turns -0 into +0).
    neg0 = np.full((2, 8), 0x80, np.uint8)
    store3 = WeightStore.open([tmp([("z", "F8_E4M3", [2, 8], neg0), ("z_scale", "F32", [0], np.zeros(0, np.float32))])])
    assert np.all(bits(store3.read("z", ctx)[1]) == 0)


def test_read_is_reference_read_with_row_sized_scale_and_six_loras(ctx, tmp):
    """The frozen `read` on a key with a shape[0]-element scale sibling and six
    stacked LoRAs (store.rs:498-515, :635-637, :732-735): bit-identical to the
    oracle's element-0 scale and merge-order FMA chain. materialize runs the
    same six deltas in the reference's order (passes of up to four through an
    f32 accumulator): f32 bit-identical, bf16 its RNE."""
    log("read: row-sized scale, six LoRAs")
    rng = np.random.default_rng(66)
    rows, cols = 96, 200
    w = synth.E4M3FN_CODES[rng.integers(0, 254, (rows, cols))]
    sc = rng.uniform(1e-3, 1e-1, rows).astype(np.float32)
    store = WeightStore.open([tmp([("m.weight", "F8_E4M3", [rows, cols], w), ("m.weight_scale", "F32", [rows], sc)])])
    ranks = [8, 16, 3, 32, 5, 64]
    dts = ["BF16", "F32", "F16", "BF16", "F8_E4M3", "BF16"]
    strengths = [1.0, 0.5, -0.75, 0.25, 2.0, 0.125]
    loras = []
    for r, dt, st in zip(ranks, dts, strengths):
        a = factor_bits(rng, dt, (r, cols), 0.05)
        b = factor_bits(rng, dt, (rows, r), 0.05)
        store.merge_lora(LoraFile.open(tmp([("m.lora_A.weight", dt, [r, cols], a),
                                            ("m.lora_B.weight", dt, [rows, r], b)])), st)
        loras.append((b.reshape(rows, r), a.reshape(r, cols), FACTOR_DT[dt], O.lora_coeff(st, None, r)))
    assert len(store.deltas("m.weight")) == 6
    want = O.read_f32(w, O.E4M3FN, O.SCALE_TENSOR, sc[:1], loras)
    assert np.array_equal(bits(store.read("m.weight", ctx)[1]), bits(want))
    want_row = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, sc, loras)
    out = ctx.alloc(rows * cols * 4)
    try:
        store.materialize(ctx, ["m.weight"], [out], lw.OUT_F32)
        got = np.empty((rows, cols), np.float32)
        ctx.download(out, got)
        assert np.array_equal(bits(got), bits(want_row))
    finally:
        ctx.free(out)
    t = store.materialize_bf16(ctx, ["m.weight"])["m.weight"]
    try:
        assert np.array_equal(t.to_numpy(), O.read_bf16(w, O.E4M3FN, O.SCALE_ROW, sc, loras))
    finally:
        t.free()


def test_multidim_empty_and_errors(ctx, tmp):
    log("multidim / empty / errors")
    rng = np.random.default_rng(8)
    w3 = synth.E4M3FN_CODES[rng.integers(0, 254, (4, 3, 5))]
    p = tmp([("c", "F8_E4M3", [4, 3, 5], w3), ("e", "F32", [0, 7], np.zeros(0, np.float32)),
             ("m.weight", "F32", [2, 3], np.zeros(6, np.float32))])
    store = WeightStore.open([p])
    got = store.read("c", ctx)[1]
    assert got.shape == (4, 3, 5)
    assert np.array_equal(bits(got).ravel(), bits(O.decode(w3.ravel(), O.E4M3FN)))
    assert store.read("e", ctx)[1].shape == (0, 7)
    # Five stacked LoRAs (more than one launch takes) all apply, in merge order.
    for k in range(5):
        store.merge_lora(LoraFile.open(tmp([("m.lora_A.weight", "F32", [1, 3], f32(1, 1, 1)),
                                            ("m.lora_B.weight", "F32", [2, 1], f32(1, k))])), 1.0)
    assert store.read("m.weight", ctx)[1].tolist() == [[5, 5, 5], [10, 10, 10]]
    with pytest.raises(lw.InvalidArgument):
        store.materialize(ctx, ["c"], [None])
    with pytest.raises(lw.MissingKey):
        store.materialize(ctx, ["c", "nope"], [1 << 12, 1 << 12])


# ---------------------------------------------------------------------------
# A synthetic DiT checkpoint (mixed formats, edge shapes, two stacked LoRAs)
# ---------------------------------------------------------------------------
def test_synthetic_block_materialise_sampled_rows(ctx, tmp_path):
    log("synthetic block: writing files")
    m, l1, l2 = (tmp_path / n for n in ("m.safetensors", "l1.safetensors", "l2.safetensors"))
    synth.write_model(m, 505, 1, variant=1, threads=8)
    synth.write_lora(l1, 506, 1, 32, variant=1, threads=8)
    synth.write_lora(l2, 507, 1, 128, variant=1, threads=8)
    store = WeightStore.open([m], KeyMap.transformer())
    store.merge_lora(LoraFile.open(l1), 1.0)
    store.merge_lora(LoraFile.open(l2), 0.5)
    layout = synth.model_layout(1, 1)
    keys = [k for k, *_ in layout]
    log("synthetic block: materialise", len(keys), "tensors")
    outs = store.materialize_bf16(ctx, keys)
    ctx.synchronize()
    try:
        for key, fmt, sm, r, c in layout:
            rows = np.unique(np.array([0, 1, 2, r // 2, r - 2, r - 1]))
            w, sc = synth.model_rows(505, key, fmt, sm, rows, c, r)
            b1, a1 = synth.lora_factors_rows(506, key, 32, rows, r, c)
            b2, a2 = synth.lora_factors_rows(507, key, 128, rows, r, c)
            case = {"w": w, "scales": sc[rows] if sm == synth.SCALE_ROW else sc, "rows": len(rows), "cols": c,
                    "fmt": fmt, "scale_mode": sm, "loras": [(b1, a1, 32, 1.0), (b2, a2, 128, 0.5)]}
            got = outs[key].to_numpy()[rows]
            stats = U.compare_lora_bf16(case, got)
            log(key, stats["max_ulp"], round(stats["frob_vs_rne_f64"], 6))
    finally:
        for t in outs.values():
            t.free()


def test_repeated_materialise_is_stable(ctx, tmp):
    """The staging and device rings are reused across calls: a second call
    with different data in the same slots gives the right answer."""
    log("repeated materialise")
    rng = np.random.default_rng(21)
    ts = []
    for k in range(6):
        w = synth.E4M3FN_CODES[rng.integers(0, 254, (128, 256))]
        ts.append((f"k{k}.weight", "F8_E4M3", [128, 256], w))
    store = WeightStore.open([tmp(ts)])
    keys = [t[0] for t in ts]
    for rep in range(3):
        order = keys if rep % 2 == 0 else keys[::-1]
        outs = store.materialize_bf16(ctx, order)
        try:
            for name, _, _, w in ts:
                assert np.array_equal(outs[name].to_numpy(), O.read_bf16(w, O.E4M3FN)), (rep, name)
        finally:
            for t in outs.values():
                t.free()


# ---------------------------------------------------------------------------
# Video-decoder value transforms (integration.rs:253-398)
# ---------------------------------------------------------------------------
def test_video_decoder_qkv_split_values(ctx, tmp):
    log("qkv split values")
    p = tmp([("vae.decoder.blocks.0.attn.qkv.weight", "F32", [3, 4], np.arange(12, dtype=np.float32))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.read("blocks.0.attn.to_q.weight", ctx)[1].tolist() == [[0, 1, 2, 3]]
    assert s.read("blocks.0.attn.to_k.weight", ctx)[1].tolist() == [[4, 5, 6, 7]]
    assert s.read("blocks.0.attn.to_v.weight", ctx)[1].tolist() == [[8, 9, 10, 11]]
    p = tmp([("vae.decoder.blocks.0.attn.qkv.weight", "F8_E4M3", [3, 1], np.array([0x38, 0x40, 0x44], np.uint8)),
             ("vae.decoder.blocks.0.attn.qkv.weight_scale", "F32", [1], f32(4.0))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert [s.read(f"blocks.0.attn.{x}.weight", ctx)[1].tolist() for x in ("to_q", "to_k", "to_v")] == [
        [[4.0]], [[8.0]], [[12.0]]]


def test_zero_type_emb_values(ctx, tmp):
    p = tmp([("vae.decoder.conv_in.weight", "F32", [2, 3, 1], np.arange(6, dtype=np.float32))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.read("type_emb", ctx)[1].tolist() == [0.0, 0.0, 0.0]


def test_video_decoder_gate_fold_values(ctx, tmp):
    log("gate fold values")
    p = tmp([("vae.decoder.blocks.0.gate_msa", "F32", [1], f32(2.0)),
             ("vae.decoder.blocks.0.attn.proj.weight", "F32", [2, 1], f32(1.0, 2.0)),
             ("vae.decoder.blocks.0.attn.proj.bias", "F32", [2], f32(0.5, 1.5))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.read("blocks.0.attn.proj.weight", ctx)[1].tolist() == [[2.0], [4.0]]
    assert s.read("blocks.0.attn.proj.bias", ctx)[1].tolist() == [1.0, 3.0]
    p = tmp([("vae.decoder.blocks.0.gate_msa", "F32", [1], f32(2.0)),
             ("vae.decoder.blocks.0.attn.proj.weight", "F8_E4M3", [1], np.array([0x38], np.uint8)),
             ("vae.decoder.blocks.0.attn.proj.weight_scale", "F32", [1], f32(4.0))])
    s = WeightStore.open([p], KeyMap.video_decoder())
    assert s.read("blocks.0.attn.proj.weight", ctx)[1].tolist() == [8.0]


def test_transforms_bit_exact_random(ctx, tmp):
    """Random FP8 / bf16 tensors through gate fold and QKV split, against the
    reference's arithmetic restated in numpy f32 (plain multiplies for the
    fold, fma(s, v, 0) for the split), with a LoRA merged onto a split part."""
    log("transforms random")
    rng = np.random.default_rng(17)
    w8 = synth.E4M3FN_CODES[rng.integers(0, 254, (6, 40))]
    w8[0, :4] = [0x80, 0x00, 0x7F, 0x01]  # -0, +0, NaN, subnormal
    wb = synth.bf16_from_f64(rng.standard_normal((12, 8)))
    s_scale, gate = np.float32(0.0371), np.float32(-1.75)
    p = tmp([("vae.decoder.m.mlp.w_down.weight", "F8_E4M3", [6, 40], w8),
             ("vae.decoder.m.mlp.w_down.weight_scale", "F32", [1], np.array([s_scale], np.float32)),
             ("vae.decoder.m.gate_mlp", "F32", [], np.array([gate], np.float32)),
             ("vae.decoder.m.attn.qkv.weight", "BF16", [12, 8], wb),
             ("vae.decoder.n.attn.qkv.weight", "F8_E4M3", [6, 40], w8),
             ("vae.decoder.n.attn.qkv.weight_scale", "F32", [1], np.array([s_scale], np.float32))])
    store = WeightStore.open([p], KeyMap.video_decoder())
    dec = O.decode(w8.ravel(), O.E4M3FN).reshape(6, 40)
    want = (dec * s_scale).astype(np.float32) * gate
    assert np.array_equal(bits(store.read("m.mlp.w_down.weight", ctx)[1]), bits(want.astype(np.float32)))
    for k, part in enumerate(("to_q", "to_k", "to_v")):
        got = store.read(f"m.attn.{part}.weight", ctx)[1]
        assert np.array_equal(bits(got), bits(O.decode(wb[4 * k:4 * k + 4].ravel(), O.BF16).reshape(4, 8)))
    # LoRA on a split FP8 part: the scaled FP8 base (fma(s, v, 0)) plus the delta, reference order.
    a = rng.normal(0, 0.05, (3, 40)).astype(np.float32)
    b = rng.normal(0, 0.05, (2, 3)).astype(np.float32)
    store.merge_lora(LoraFile.open(tmp([("n.attn.to_k.lora_A.weight", "F32", [3, 40], a),
                                        ("n.attn.to_k.lora_B.weight", "F32", [2, 3], b)])), 0.5)
    want = O.read_f32(w8[2:4], O.E4M3FN, O.SCALE_TENSOR, np.array([s_scale], np.float32),
                      [(b, a, O.F32, O.lora_coeff(0.5, None, 3))])
    assert np.array_equal(bits(store.read("n.attn.to_k.weight", ctx)[1]), bits(want))


# ---------------------------------------------------------------------------
# Device hand-off: materialise into a consumer framework's own tensors
# ---------------------------------------------------------------------------
def test_dlpack_export_of_materialised_tensor(ctx, tmp):
    """A materialised tensor exports a DLPack capsule over its own HBM (no
    copy): ROCm device, bf16, row-major shape and strides, and the data the
    capsule points at is the materialised result."""
    from ltx_weights import _dlpack
    log("dlpack export")
    case = synth.tensor_case(31, 256, 512, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
    store = WeightStore.open([tmp([("l.weight", "F8_E4M3", [256, 512], case["w"]),
                                   ("l.weight_scale", "F32", [256], case["scales"])])])
    t = store.materialize_bf16(ctx, ["l.weight"])["l.weight"]
    try:
        assert t.__dlpack_device__() == (_dlpack.KDL_ROCM, 0)
        cap = t.__dlpack__()
        mt = _dlpack.view(cap)
        dl = mt.dl_tensor
        assert dl.data == t.ptr and dl.ndim == 2 and dl.byte_offset == 0
        assert (dl.device.device_type, dl.device.device_id) == (_dlpack.KDL_ROCM, 0)
        assert (dl.dtype.code, dl.dtype.bits, dl.dtype.lanes) == (_dlpack.KDL_BFLOAT, 16, 1)
        assert [dl.shape[0], dl.shape[1]] == [256, 512] and [dl.strides[0], dl.strides[1]] == [512, 1]
        out = np.empty((256, 512), np.uint16)
        ctx.download(dl.data, out)
        assert np.array_equal(out, O.read_bf16(case["w"], O.E4M3FN, O.SCALE_ROW, case["scales"]))
        mt.deleter(ctypes.pointer(mt))  # the consumer's release
    finally:
        t.free()


def test_materialised_weight_consumed_in_place_by_rocblas_gemm(ctx, tmp):
    """The hand-off to a consumer: rocBLAS (the system ROCm runtime, as a
    Burn HIP backend would use) runs y = x W^T straight on the bf16 buffer
    that materialize wrote, through the DLPack capsule's data pointer and on
    the library's compute stream, as ltx-dit's load_linear transposes the
    [out, in] weight (crates/ltx-dit/src/load.rs:149-170) and multiplies.
    The GEMM's f32 output must match the f64 product of the same bf16
    weights within the f32 GEMM error bound."""
    from ltx_weights import _dlpack
    log("hand-off: rocBLAS GEMM on the materialised buffer")
    try:
        rb = ctypes.CDLL("librocblas.so")
    except OSError:
        pytest.skip("librocblas.so not found")
    rows, cols, batch = 384, 1024, 16
    case = synth.tensor_case(77, rows, cols, synth.E4M3FN, synth.SCALE_ROW, loras=((64, 1.0),))
    b, a, r, c = case["loras"][0]
    store = WeightStore.open([tmp([("l.weight", "F8_E4M3", [rows, cols], case["w"]),
                                   ("l.weight_scale", "F32", [rows], case["scales"])])])
    store.merge_lora(LoraFile.open(tmp([("l.lora_A.weight", "BF16", [r, cols], a),
                                        ("l.lora_B.weight", "BF16", [rows, r], b)])), c)
    t = store.materialize_bf16(ctx, ["l.weight"])["l.weight"]
    rng = np.random.default_rng(5)
    x = synth.bf16_from_f64(rng.normal(0.0, 1.0, size=(batch, cols)))
    px = ctx.alloc(x.nbytes)
    py = ctx.alloc(batch * rows * 4)
    handle = ctypes.c_void_p()
    try:
        cap = t.__dlpack__()  # held until the consumer's release below
        mt = _dlpack.view(cap)
        w_ptr = mt.dl_tensor.data
        ctx.upload(x, px)
        vp = ctypes.c_void_p
        rb.rocblas_create_handle.argtypes = [ctypes.POINTER(vp)]
        rb.rocblas_set_stream.argtypes = [vp, vp]
        rb.rocblas_destroy_handle.argtypes = [vp]
        i32 = ctypes.c_int
        rb.rocblas_gemm_ex.argtypes = [vp, i32, i32, i32, i32, i32, vp, vp, i32, i32, vp, i32, i32, vp, vp, i32, i32,
                                       vp, i32, i32, i32, i32, ctypes.c_int32, ctypes.c_uint32]
        assert rb.rocblas_create_handle(ctypes.byref(handle)) == 0
        assert rb.rocblas_set_stream(handle, ctx.stream()) == 0
        alpha, beta = ctypes.c_float(1.0), ctypes.c_float(0.0)
        none, trans, bf16, f32_ = 111, 112, 168, 151
        # Column-major view: Y^T [rows x batch] = W [rows x cols] * X^T [cols x batch]; the
        # row-major [rows, cols] weight is the column-major [cols x rows] matrix W^T.
        st = rb.rocblas_gemm_ex(handle, trans, none, rows, batch, cols, ctypes.byref(alpha), w_ptr, bf16, cols,
                                px, bf16, cols, ctypes.byref(beta), py, f32_, rows, py, f32_, rows, f32_, 0, 0, 0)
        assert st == 0, f"rocblas_gemm_ex status {st}"
        ctx.synchronize()
        y = np.empty((batch, rows), np.float32)
        ctx.download(py, y)
        w64 = U.bf16_to_f64(t.to_numpy())
        x64 = U.bf16_to_f64(x)
        ref = x64 @ w64.T
        bound = (cols + 2) * 2.0 ** -24 * (np.abs(x64) @ np.abs(w64).T)
        assert np.all(np.abs(y - ref) <= bound), float(np.max(np.abs(y - ref) / np.maximum(bound, 1e-300)))
        # and the weight the GEMM read is the library's result
        U.compare_lora_bf16(case, t.to_numpy())
        mt.deleter(ctypes.pointer(mt))
    finally:
        if handle.value:
            rb.rocblas_destroy_handle(handle)
        ctx.free(px)
        ctx.free(py)
        t.free()


def test_exact_materialise_of_synthetic_block(ctx, tmp_path):
    """LTXW_MAT_EXACT: a DiT block (two stacked bf16 LoRAs, mixed formats)
    bit-identical to the reference order on sampled rows."""
    log("exact materialise: writing files")
    m, l1, l2 = (tmp_path / n for n in ("m.safetensors", "l1.safetensors", "l2.safetensors"))
    synth.write_model(m, 705, 1, variant=1, threads=8)
    synth.write_lora(l1, 706, 1, 32, variant=1, threads=8)
    synth.write_lora(l2, 707, 1, 128, variant=1, threads=8)
    store = WeightStore.open([m], KeyMap.transformer())
    store.merge_lora(LoraFile.open(l1), 1.0)
    store.merge_lora(LoraFile.open(l2), 0.5)
    layout = synth.model_layout(1, 1)
    keys = [k for k, *_ in layout]
    outs = {}
    try:
        for k, (key, fmt, sm, r, c) in enumerate(layout):
            outs[key] = ctx.alloc(2 * r * c)
        store.materialize(ctx, keys, [outs[k] for k in keys], lw.OUT_BF16, MAT_EXACT)
        for key, fmt, sm, r, c in layout[7:]:
            rows = np.array([0, r // 2, r - 1])
            w, sc = synth.model_rows(705, key, fmt, sm, rows, c, r)
            b1, a1 = synth.lora_factors_rows(706, key, 32, rows, r, c)
            b2, a2 = synth.lora_factors_rows(707, key, 128, rows, r, c)
            full = np.empty((r, c), np.uint16)
            ctx.download(outs[key], full)
            ref = O.read_bf16(w, U.FMT_TO_ORC[fmt], sm, sc[rows] if sm == synth.SCALE_ROW else sc,
                              [(b1, a1, O.BF16, O.lora_coeff(1.0, None, 32)),
                               (b2, a2, O.BF16, O.lora_coeff(0.5, None, 128))])
            assert np.array_equal(full[rows], ref), key
    finally:
        for p in outs.values():
            ctx.free(p)


def test_mixed_factor_types_on_one_tensor(ctx, tmp):
    """A bf16 adapter and an f32 adapter stacked on one key: reference order,
    bit-exact (the exact kernel reads each LoRA's own element type)."""
    log("mixed factor types")
    rng = np.random.default_rng(23)
    rows, cols = 96, 136
    w = synth.E4M3FN_CODES[rng.integers(0, 254, (rows, cols))]
    sc = rng.uniform(1e-3, 1e-1, rows).astype(np.float32)
    store = WeightStore.open([tmp([("x.weight", "F8_E4M3", [rows, cols], w), ("x.weight_scale", "F32", [rows], sc)])])
    a1, b1 = factor_bits(rng, "BF16", (16, cols), 0.05), factor_bits(rng, "BF16", (rows, 16), 0.05)
    a2, b2 = factor_bits(rng, "F32", (8, cols), 0.05), factor_bits(rng, "F32", (rows, 8), 0.05)
    store.merge_lora(LoraFile.open(tmp([("x.lora_A.weight", "BF16", [16, cols], a1),
                                        ("x.lora_B.weight", "BF16", [rows, 16], b1)])), 1.0)
    store.merge_lora(LoraFile.open(tmp([("x.lora_A.weight", "F32", [8, cols], a2),
                                        ("x.lora_B.weight", "F32", [rows, 8], b2)])), 0.5)
    want = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, sc, [(b1, a1, O.BF16, O.lora_coeff(1.0, None, 16)),
                                                     (b2, a2, O.F32, O.lora_coeff(0.5, None, 8))])
    assert np.array_equal(bits(store.read("x.weight", ctx, flags=MAT_ROW_SCALES)[1]), bits(want))


def test_materialise_small_staging_slots_many_tensors(tmp):
    """Staging slots of 12 KiB: pieces of the batch layout span several small
    tensors (scales and factors included) and large tensors span several
    pieces. Every tensor must come out as the oracle's: bit-exact on the
    reference-order paths, within tolerance on the MFMA path."""
    log("small staging slots")
    rng = np.random.default_rng(31)
    spec = [  # key, base dtype, shape, scale, LoRA rank (bf16 file) or None, f16 LoRA rank or None
        ("a", "F8_E4M3", (64, 256), "row", 16, None),
        ("b", "F8_E5M2", (3, 8), "tensor", None, None),
        ("c", "BF16", (20, 40), None, None, None),
        ("d", "F8_E4M3", (100, 72), "row", 8, None),
        ("e", "F32", (7, 9), None, None, 2),
        ("f", "F8_E4M3", (1, 8), None, None, None),
        ("g", "F8_E5M2", (130, 264), "row", 32, None),
        ("h", "F8_E4M3", (5, 4104), "tensor", None, None),
        ("i", "F16", (33, 17), None, 4, None),
    ]
    ts, l1, l2, info = [], [], [], {}
    for key, dt, (rows, cols), scale, r1, r2 in spec:
        w = base_bits(rng, dt, (rows, cols))
        ts.append((f"{key}.weight", dt, [rows, cols], w))
        sc = None
        if scale == "row":
            sc = rng.uniform(1e-3, 1e-1, rows).astype(np.float32)
            ts.append((f"{key}.weight_scale", "F32", [rows], sc))
        elif scale == "tensor":
            sc = rng.uniform(1e-3, 1e-1, 1).astype(np.float32)
            ts.append((f"{key}.weight_scale", "F32", [], sc))
        loras = []
        for files, r, fdt, strength in ((l1, r1, "BF16", 1.0), (l2, r2, "F16", 0.75)):
            if r is None:
                continue
            a = factor_bits(rng, fdt, (r, cols), 0.05)
            b = factor_bits(rng, fdt, (rows, r), 0.05)
            files += [(f"{key}.lora_A.weight", fdt, [r, cols], a), (f"{key}.lora_B.weight", fdt, [rows, r], b)]
            loras.append((b.reshape(rows, r), a.reshape(r, cols), FACTOR_DT[fdt], O.lora_coeff(strength, None, r)))
        info[key] = (w.reshape(rows, cols), dt, scale, sc, loras)
    store = WeightStore.open([tmp(ts)])
    store.merge_lora(LoraFile.open(tmp(l1)), 1.0)
    store.merge_lora(LoraFile.open(tmp(l2)), 0.75)
    keys = [f"{k}.weight" for k, *_ in spec]
    with lw.Context(0, staging_bytes=12288, n_staging=3) as small:
        outs = store.materialize_bf16(small, keys)
        try:
            for key, dt, (rows, cols), scale, r1, r2 in spec:
                w, dt, scale, sc, loras = info[key]
                got = outs[f"{key}.weight"].to_numpy()
                smode = {None: O.SCALE_NONE, "row": O.SCALE_ROW, "tensor": O.SCALE_TENSOR}[scale]
                mfma = r1 is not None and r2 is None and dt.startswith("F8") and cols % 8 == 0
                if mfma:
                    case = {"w": w, "scales": sc, "rows": rows, "cols": cols, "scale_mode": smode,
                            "fmt": synth.E4M3FN if dt == "F8_E4M3" else synth.E5M2,
                            "loras": [(b, a, b.shape[1], c) for (b, a, _, c) in loras]}
                    U.compare_lora_bf16(case, got)
                else:
                    want = O.read_bf16(w, O.DTYPE_CODES[dt], smode, sc, loras)
                    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), key
        finally:
            for t in outs.values():
                t.free()


@pytest.mark.parametrize("base_dt", ["BF16", "F16"])
@pytest.mark.parametrize("ranks,shape", [([64], (256, 512)), ([32, 16], (130, 264))])
def test_16bit_base_fused_path(ctx, tmp, base_dt, ranks, shape):
    """bf16 / f16 bases with bf16 LoRAs run on the several-LoRA MFMA kernel:
    within the fused tolerance of the oracle by default, bit-exact with
    MAT_EXACT."""
    log("16-bit base fused", base_dt, ranks, shape)
    rng = np.random.default_rng(77 + len(ranks))
    rows, cols = shape
    w = base_bits(rng, base_dt, (rows, cols))
    store = WeightStore.open([tmp([("t.weight", base_dt, [rows, cols], w)])])
    loras = []
    for k, r in enumerate(ranks):
        a = factor_bits(rng, "BF16", (r, cols), 0.05)
        b = factor_bits(rng, "BF16", (rows, r), 0.05)
        strength = [1.0, 0.5][k]
        store.merge_lora(LoraFile.open(tmp([("t.lora_A.weight", "BF16", [r, cols], a),
                                            ("t.lora_B.weight", "BF16", [rows, r], b)])), strength)
        loras.append((b.reshape(rows, r), a.reshape(r, cols), O.lora_coeff(strength, None, r)))
    case = {"w": w.reshape(rows, cols), "scales": None, "rows": rows, "cols": cols, "scale_mode": O.SCALE_NONE,
            "fmt": {"BF16": lw.FMT_BF16, "F16": lw.FMT_F16}[base_dt],
            "loras": [(b, a, b.shape[1], c) for (b, a, c) in loras]}
    out = store.materialize_bf16(ctx, ["t.weight"], flags=MAT_MFMA)["t.weight"]
    try:
        U.compare_lora_bf16(case, out.to_numpy())
    finally:
        out.free()
    want = O.read_bf16(case["w"], O.DTYPE_CODES[base_dt], O.SCALE_NONE, None,
                       [(b, a, O.BF16, c) for (b, a, c) in loras])
    for flags in (0, MAT_EXACT):  # the default is the reference's order
        out = store.materialize_bf16(ctx, ["t.weight"], flags=flags)["t.weight"]
        try:
            assert np.array_equal(out.to_numpy(), want)
        finally:
            out.free()
    out = store.materialize_bf16(ctx, ["t.weight"], flags=MAT_EXACT)["t.weight"]
    try:
        assert np.array_equal(out.to_numpy(), want)
    finally:
        out.free()
