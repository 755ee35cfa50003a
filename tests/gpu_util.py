"""Helpers for the GPU parity tests: run a case through the C ABI and compare
it with the CPU oracle under the stated tolerances."""
import os

import numpy as np

import ltx_weights as lw
import oracle_lib as O

FMT_TO_ORC = {lw.FMT_E4M3FN: O.E4M3FN, lw.FMT_E5M2: O.E5M2, lw.FMT_BF16: O.BF16, lw.FMT_F16: O.F16}
# LoRA factor element types (a case's LoRA tuples are (B, A, rank, coeff) or
# (B, A, rank, coeff, factor type); bf16 when absent).
FDT_TO_ORC = {lw.FACTOR_BF16: O.BF16, lw.FACTOR_F32: O.F32, lw.FACTOR_F16: O.F16,
              lw.FACTOR_E4M3FN: O.E4M3FN, lw.FACTOR_E5M2: O.E5M2}


def lora_fdt(lo):
    return lo[4] if len(lo) > 4 else lw.FACTOR_BF16


class Dev:
    """Device copies of one case's inputs plus an output buffer."""

    def __init__(self, ctx, case, out_dtype=lw.OUT_BF16, w_offset=0, out_offset=0):
        self.ctx = ctx
        self.case = case
        self.out_dtype = out_dtype
        self.ptrs = []
        rows, cols = case["rows"], case["cols"]
        n = rows * cols
        self.w_base = self._put(case["w"], extra=w_offset)
        self.w = self.w_base + w_offset
        self.s = self._put(case["scales"]) if case["scales"] is not None else None
        self.loras = []
        for lo in case["loras"]:
            b, a, rank, coeff = lo[:4]
            self.loras.append((self._put(b), self._put(a), rank, coeff, lora_fdt(lo)))
        ob = 4 if out_dtype == lw.OUT_F32 else 2
        self.out_base = ctx.alloc(max(1, n * ob + out_offset + 64))
        self.ptrs.append(self.out_base)
        self.out = self.out_base + out_offset
        self.n = n
        self.ob = ob

    def _put(self, arr, extra=0):
        arr = np.ascontiguousarray(arr)
        p = self.ctx.alloc(max(1, arr.nbytes + extra + 64))
        self.ptrs.append(p)
        if arr.nbytes:
            self.ctx.upload(arr, p + extra)
        return p

    def run(self):
        c = self.case
        if c["loras"]:
            self.ctx.dequant_lora(self.w, c["rows"], c["cols"], c["fmt"], c["scale_mode"], self.s,
                                  self.loras, self.out, self.out_dtype)
        else:
            self.ctx.dequant(self.w, c["rows"], c["cols"], c["fmt"], c["scale_mode"], self.s,
                             self.out, self.out_dtype)

    def result(self):
        dt = np.float32 if self.out_dtype == lw.OUT_F32 else np.uint16
        out = np.empty((self.case["rows"], self.case["cols"]), dtype=dt)
        self.ctx.download(self.out, out)
        return out

    def free(self):
        for p in self.ptrs:
            self.ctx.free(p)
        self.ptrs = []


def oracle_args(case, row_sel=None):
    """Oracle inputs, optionally restricted to a subset of output rows (rows
    are independent: row o needs W[o], scale[o] and B[o] only)."""
    w, s = case["w"], case["scales"]
    loras = [(lo[0], lo[1], FDT_TO_ORC[lora_fdt(lo)], lo[3]) for lo in case["loras"]]
    if row_sel is not None:
        w = w[row_sel]
        if s is not None and case["scale_mode"] == lw.SCALE_ROW:
            s = s[row_sel]
        loras = [(b[row_sel], a, dt, c) for (b, a, dt, c) in loras]
    return w, FMT_TO_ORC[case["fmt"]], case["scale_mode"], s, loras


def oracle_bf16(case, row_sel=None, threads=16):
    w, f, m, s, loras = oracle_args(case, row_sel)
    return O.read_bf16(w, f, m, s, loras, threads=threads)


def oracle_f32(case, row_sel=None, threads=16):
    w, f, m, s, loras = oracle_args(case, row_sel)
    return O.read_f32(w, f, m, s, loras, threads=threads)


def bf16_ordered(u16):
    """Monotone integer image of bf16 bit patterns; +0 and -0 both map to 0."""
    u = u16.astype(np.int32)
    return np.where(u & 0x8000, -(u & 0x7FFF), u)


def bf16_to_f64(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


# Statistics of every compare_lora_bf16 call in this process, in call order
# (the GPU test session writes them out; see conftest.py).
STATS = []


def compare_lora_bf16(case, got, row_sel=None, label=None):
    """Tolerance for the fused path (MFMA summation order differs from the
    reference's sequential FMA chain):
      (1) every element within 1 bf16 ulp (ordered distance) of the
          reference's own result RNE(reference f32), except
      (2) elements further away than that which are no farther from the
          exact value W64 (f64 sum of the same terms) than the reference's
          f32 is: |gpu - W64| <= |ref32 - W64| (the reference's own chain
          lost more than a bf16 step to rounding), and
      (3) ill-conditioned elements (catastrophic cancellation, |W64| a tiny
          fraction of S = |deq| + sum |c B A|) where neither order is
          accurate: these must lie within the f32 forward-error bound that
          the f32-output tests use, |gpu - W64| <= (K + 4) 2^-24 S plus the
          bf16 rounding of the result (2^-8 |gpu|), K the total rank. The
          reference's chain meets the same bound; the matrix cores' order
          can land farther from W64 than the chain does in such an element
          (their products are aligned to the largest one of each 32-term
          group before the sum). Their count is reported (n_cond) and is a
          few per 10^7 elements on random factors;
      (4) ||out - RNE(W64)||_F / ||W64||_F <= 1e-3 (Frobenius, against the
          bf16-rounded f64 oracle; bf16 rounding alone is ~1.7e-3 against the
          unrounded value, which is reported too).
    NaN positions and encodings must match exactly. The bit-identical
    alternative is the exact kernel (MAT_EXACT), tested separately.
    Returns a dict of statistics (also appended to STATS); raises
    AssertionError on failure."""
    ref32 = oracle_f32(case, row_sel)
    ref = O.read_bf16(ref32, O.F32, threads=16)
    got = np.asarray(got)
    nan_r = np.isnan(bf16_to_f64(ref))
    nan_g = np.isnan(bf16_to_f64(got))
    assert np.array_equal(nan_r, nan_g), "NaN positions differ"
    assert np.array_equal(ref[nan_r], got[nan_g]), "NaN encodings differ"
    d = np.abs(bf16_ordered(got) - bf16_ordered(ref))
    d[nan_r] = 0
    bad = d > 1
    stats = {"n": int(got.size), "max_ulp": int(d.max()) if d.size else 0, "n_over_1ulp": int(bad.sum()),
             "label": label or case.get("label") or os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0], "shape": [int(x) for x in got.shape]}
    STATS.append(stats)
    w, f, m, s, loras = oracle_args(case, row_sel)
    w64 = O.read_f64_rows(w, f, m, s, loras)
    g64 = bf16_to_f64(got)
    if bad.any():
        err_gpu = np.abs(g64 - w64)
        err_ref = np.abs(ref32.astype(np.float64) - w64)
        worse = bad & ~(err_gpu <= err_ref)
        stats["n_cond"] = int(worse.sum())
        stats["over_1ulp"] = [
            {"flat": int(k), "gpu": int(got.flat[k]), "ref_bf16": int(ref.flat[k]),
             "err_gpu": float(err_gpu.flat[k]), "err_ref32": float(err_ref.flat[k])}
            for k in np.flatnonzero(bad)[:8]]
        if worse.any():
            k_rank = sum(int(lo[2]) for lo in case["loras"])
            cols = got.shape[-1]
            bound = np.zeros(got.shape, dtype=np.float64)
            for r in np.unique(np.flatnonzero(worse) // cols):
                bound[r] = O.abs_bound_rows(w, f, m, s, loras, row0=int(r), nrows=1)[0]
            lim = (k_rank + 4) * 2.0 ** -24 * bound + 2.0 ** -8 * np.abs(g64)
            ratio = np.where(worse, err_gpu / np.maximum(lim, 1e-300), 0.0)
            stats["cond_err_over_limit"] = float(ratio.max())
            stats["cond_y_over_S"] = float(np.max(np.where(worse, np.abs(w64) / np.maximum(bound, 1e-300), 0.0)))
            assert ratio.max() <= 1.0, (
                "%d elements beyond 1 ulp of the reference, farther from the exact value than its f32 and outside "
                "the f32 forward-error bound (%s)" % (int((ratio > 1).sum()), stats["over_1ulp"]))
    fin = np.isfinite(w64) & np.isfinite(g64)
    r64 = bf16_to_f64(bf16_from_f64_exact(w64))
    den = np.linalg.norm(w64[fin])
    stats["frob_vs_rne_f64"] = float(np.linalg.norm(g64[fin] - r64[fin]) / den) if den else 0.0
    stats["frob_vs_f64"] = float(np.linalg.norm(g64[fin] - w64[fin]) / den) if den else 0.0
    assert stats["frob_vs_rne_f64"] <= 1e-3, stats
    return stats


def bf16_from_f64_exact(x):
    from ltx_weights.synth import bf16_from_f64
    out = np.zeros(x.shape, dtype=np.uint16)
    fin = np.isfinite(x)
    out[fin] = bf16_from_f64(x[fin])
    return out
