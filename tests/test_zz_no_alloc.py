"""ltxw_dequant_lora_grouped_noalloc (the allocation-free grouped call)
against ltxw_dequant_lora_grouped through the C ABI: the same kernels, so
the outputs must be bit-identical, on two calls in a row (the second one
smaller, so that it runs on a scratch array the first call left full), and
a call over the descriptor limit must be refused before anything runs."""
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


def tensor_set(seed, big):
    """Descriptor specs: several single-LoRA jobs, several two-LoRA jobs (the
    several-LoRA kernel), f32 outputs, a plain dequant, a reference-order
    (exact) tensor, and enough small rank-64 tensors (30, or 25 in the small
    set) that their launch's job records exceed what the kernel arguments
    carry, so that launch reads them from the scratch array."""
    s = 2 if big else 1
    specs = [
        (256 * s, 512 * s, ((64, 1.0),), lw.OUT_BF16, 0),
        (300 * s, 520, ((64, 0.5),), lw.OUT_BF16, 0),
        (128, 264 * s, ((64, 1.5),), lw.OUT_BF16, 0),
        (257, 1032, ((32, 1.0), (128, 0.5)), lw.OUT_BF16, 0),
        (512 * s, 256, ((32, 1.0), (128, 0.5)), lw.OUT_BF16, 0),
        (256, 384 * s, ((64, 1.0),), lw.OUT_F32, 0),
        (130, 520, ((64, 1.0),), lw.OUT_F32, 0),
        (200 * s, 328, (), lw.OUT_BF16, 0),
        (96, 264, ((16, 1.0),), lw.OUT_BF16, lw.DESC_EXACT),
    ]
    if not big:
        specs = specs[1:5] + specs[6:8]
    specs += [(64 + 8 * (k % 3), 128, ((64, 1.0),), lw.OUT_BF16, 0) for k in range(30 if big else 25)]
    cases = []
    for k, (rows, cols, loras, out_dtype, flags) in enumerate(specs):
        fmt = synth.E5M2 if k % 3 == 1 else synth.E4M3FN
        sm = synth.SCALE_ROW if k % 2 == 0 else synth.SCALE_TENSOR
        c = synth.tensor_case(seed + k, rows, cols, fmt, sm, loras=loras)
        cases.append((c, out_dtype, flags))
    return cases


def run_both(ctx, cases):
    """Uploads the cases, runs them through both calls into separate outputs
    and returns (grouped outputs, noalloc outputs) as host arrays."""
    devs, da, db = [], [], []
    try:
        for c, out_dtype, flags in cases:
            d = U.Dev(ctx, c, out_dtype)
            devs.append(d)
            ob = ctx.alloc(max(1, c["rows"] * c["cols"] * d.ob + 64))
            d.ptrs.append(ob)
            ctx.memset(d.out, 0x5A, c["rows"] * c["cols"] * d.ob)
            ctx.memset(ob, 0xA5, c["rows"] * c["cols"] * d.ob)
            base = {"w": d.w, "scales": d.s, "rows": c["rows"], "cols": c["cols"], "fmt": c["fmt"],
                    "scale_mode": c["scale_mode"], "out_dtype": out_dtype, "flags": flags, "loras": d.loras}
            da.append(dict(base, out=d.out))
            db.append(dict(base, out=ob))
        ctx.grouped(da)
        ctx.grouped_noalloc(db)
        ctx.synchronize()
        outs_a, outs_b = [], []
        for (c, out_dtype, _), d, b in zip(cases, devs, db):
            dt = np.float32 if out_dtype == lw.OUT_F32 else np.uint16
            a_host = np.empty((c["rows"], c["cols"]), dtype=dt)
            b_host = np.empty_like(a_host)
            ctx.download(d.out, a_host)
            ctx.download(b["out"], b_host)
            outs_a.append(a_host)
            outs_b.append(b_host)
        return outs_a, outs_b
    finally:
        for d in devs:
            d.free()


@pytest.mark.parametrize("calls", [("big", "small")])
def test_noalloc_matches_grouped_two_calls(ctx, calls):
    for seed, size in zip((700, 800), calls):
        cases = tensor_set(seed, size == "big")
        log("case: noalloc vs grouped,", size, len(cases), "tensors")
        outs_a, outs_b = run_both(ctx, cases)
        for k, ((c, out_dtype, _), a, b) in enumerate(zip(cases, outs_a, outs_b)):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{size} call, tensor {k} differs"
        # The shared result is the library's: within the fused path's bar of the oracle.
        c0, _, _ = cases[0]
        sel = np.unique(np.linspace(0, c0["rows"] - 1, 16).astype(np.int64))
        U.compare_lora_bf16(c0, outs_b[0][sel], row_sel=sel)


def test_noalloc_refuses_too_many_descriptors(ctx):
    log("case: noalloc over the descriptor limit")
    c = synth.tensor_case(900, 128, 128, synth.E4M3FN, synth.SCALE_ROW, loras=((16, 1.0),))
    d = U.Dev(ctx, c)
    try:
        ctx.memset(d.out, 0x5A, 128 * 128 * 2)
        desc = {"w": d.w, "scales": d.s, "rows": 128, "cols": 128, "fmt": c["fmt"], "scale_mode": c["scale_mode"],
                "out": d.out, "loras": d.loras}
        with pytest.raises(lw.InvalidArgument):
            ctx.grouped_noalloc([desc] * (lw.NOALLOC_MAX_DESCS + 1))
        ctx.synchronize()
        out = d.result()
        assert np.all(out == 0x5A5A), "a refused call queued work"
        ctx.grouped_noalloc([desc] * lw.NOALLOC_MAX_DESCS)  # at the limit: runs
        ctx.synchronize()
        U.compare_lora_bf16(c, d.result())
    finally:
        d.free()
