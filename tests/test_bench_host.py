"""CPU checks of bench.py's host-side setup: every device pointer a grouped
descriptor carries must point at a buffer of exactly the size the kernels
read for that tensor (weight, scales, LoRA B, LoRA A, output). A mistake
here would make a kernel read past an allocation on the GPU."""
import importlib.util
import os

import pytest

from ltx_weights import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def load_bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


class MockCtx:
    def __init__(self):
        self.next = 1 << 20
        self.size = {}
        self.uploaded = {}

    def alloc(self, n):
        p = self.next
        self.next += ((max(n, 1) + 255) // 256) * 256 + 4096
        self.size[p] = n
        return p

    def upload(self, x, p):
        assert x.nbytes == self.size[p]
        self.uploaded[p] = x


class MockHip:
    def __init__(self, ctx):
        self.ctx = ctx

    def copy_d2d(self, dst, src, n, stream):
        assert self.ctx.size[dst] == n == self.ctx.size[src]


@pytest.mark.parametrize("workload", ["layer", "dequant", "block", "mixed"])
def test_descriptors_point_at_correctly_sized_buffers(workload):
    bench = load_bench()
    small = {"layer": (256, 512), "dequant": (128, 256), "block": None, "mixed": None}

    # Shrink shapes so the check runs fast; the indexing logic is shape-independent.
    def shrink(name, s):
        cases = bench.workload_cases(name, s)
        out = []
        for c in cases:
            r, co = (c["rows"] // 32, c["cols"] // 32)
            ranks = tuple((l[2], l[3]) for l in c["loras"])
            out.append(synth.tensor_case(7, r, co, c["fmt"], c["scale_mode"], loras=ranks))
        return out

    cases = shrink(workload, synth)
    ctx = MockCtx()
    insts, allocs, n = bench.build_instances(ctx, cases, MockHip(ctx), None, rotate_bytes=1)
    assert n == 2 and len(insts) == 2
    for descs in insts:
        for c, d in zip(cases, descs):
            rows, cols = c["rows"], c["cols"]
            assert ctx.size[d["w"]] == rows * cols
            assert ctx.size[d["out"]] == rows * cols * 2
            if c["scale_mode"] == synth.SCALE_ROW:
                assert ctx.size[d["scales"]] == 4 * rows
            elif c["scale_mode"] == synth.SCALE_TENSOR:
                assert ctx.size[d["scales"]] == 4
            else:
                assert d["scales"] is None
            assert len(d["loras"]) == len(c["loras"])
            for (b_p, a_p, r, co), (b, a, r2, co2) in zip(d["loras"], c["loras"]):
                assert (r, co) == (r2, co2)
                assert ctx.size[b_p] == rows * r * 2 and ctx.size[a_p] == r * cols * 2
    # the first instance uploads the host arrays themselves
    for c, d in zip(cases, insts[0]):
        assert ctx.uploaded[d["w"]] is c["w"]
        for (b_p, a_p, _, _), (b, a, _, _) in zip(d["loras"], c["loras"]):
            assert ctx.uploaded[b_p] is b and ctx.uploaded[a_p] is a
