"""Benchmark: fused FP8 dequant + LoRA merge on one MI355X.

Headline workload ("layer"; one step = one fused dequant + merge of one DiT
linear layer):
  W 4096 (out) x 4096 (in) e4m3fn, per-output-row f32 scales U[1e-3, 1e-1],
  LoRA B 4096 x 64 and A 64 x 4096 bf16 ~ N(0, 0.02^2), alpha = 1, bf16 out.
Measured beside it in the same run (--configs): "dequant" (4096 x 4096
e4m3fn, one scale, no LoRA), "block" (one DiT block of 10 tensors in one
grouped launch), "mixed" (e5m2 FFN / e4m3fn attention, two stacked LoRAs
r32 + r128, 4096x4104 and 4104x16384 edge tensors), the streaming-dequant
ceiling of the same 1 B in / 2 B out pattern, and whole-model
materialisation from safetensors files (--e2e). Kernel inputs are resident
in HBM before timing; consecutive steps rotate over >= 1 GiB of distinct
buffers so the 256 MB MALL cannot serve repeats; after the warmup and a
synchronize, 200 ms of large dequant launches (--lead-ms) run ahead of the
timed steps, so that those start with the GPU in its loaded steady state and
run back to back on the GPU whatever the host's submission rate (also under a
profiler).

value     = algorithmic bytes per step * steps / timed seconds (GB/s), with
            algorithmic bytes = out*in (FP8) + 2*out*in (bf16 out) + scale
            bytes + 2*r*(out+in) (bf16 factors) per tensor, timed with HIP
            events on the library's compute stream (the stream the kernels run on).
roofline  = that figure against MI355X's 8 TB/s HBM peak; `traffic` is the
            rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the
            same counter on a plain device copy, from profiles/ when present.
cpu_baseline = the CPU oracle (a C restatement of the reference's read path,
            same operation order) on the workload's first tensor, host cores.

Prints exactly one JSON line on stdout; progress goes to stderr.
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "ltx-rust_amd"))

import numpy as np  # noqa: E402

METRIC = "dequant+LoRA-merge GB/s & % HBM roofline; s to materialise 22B weights"
HBM_PEAK_GBPS = 8000.0
ROWS, COLS, RANK = 4096, 4096, 64
ROTATE_BYTES = 1 << 30
PARITY_BAR = ("gpu_util.compare_lora_bf16: each element <= 1 bf16 ulp of the reference's result, or no farther "
              "from the exact (f64) value than the reference's f32, or (n_cond, ill-conditioned) within the f32 "
              "forward-error bound (K+4) 2^-24 (|deq| + sum|cBA|) + bf16 rounding; Frobenius <= 1e-3")
PMC_SUMMARY = {
    "layer": os.path.join(ROOT, "profiles", "k_fused_pair_layer4096x4096_r64.pmc.txt"),
    "block": os.path.join(ROOT, "profiles", "k_fused_pair_ditblock_r64.pmc.txt"),
    "dequant": os.path.join(ROOT, "profiles", "k_dequant_tile_layer4096x4096.pmc.txt"),
    "mixed": os.path.join(ROOT, "profiles", "k_fused_pair_multi_mixedblock_r32_r128.pmc.txt"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Hip:
    """The few HIP runtime calls the bench needs (events, device copies)."""

    def __init__(self):
        self.L = ctypes.CDLL("libamdhip64.so")
        self.L.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.L.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.L.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.L.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.L.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_void_p]

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with HIP error {rc}")

    def event(self):
        e = ctypes.c_void_p()
        self._ok(self.L.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def record(self, e, stream):
        self._ok(self.L.hipEventRecord(e, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self._ok(self.L.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self._ok(self.L.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value

    def copy_d2d(self, dst, src, n, stream):
        self._ok(self.L.hipMemcpyAsync(dst, src, n, 3, stream), "hipMemcpyAsync D2D")


def read_traffic(workload):
    """Per-dispatch HBM bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated
    against a plain device copy) from the committed summary for `workload`."""
    path = PMC_SUMMARY.get(workload)
    if not path or not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and line.strip().startswith("traffic_bytes_per_dispatch"):
                try:
                    vals["traffic"] = float(line.split(":", 1)[1].split()[0])
                except ValueError:
                    pass
    return vals.get("traffic")


def cpu_baseline(case, budget_s, threads=None):
    """The oracle on the same tensor, `threads` host threads (default all, at
    most 16), repeated to ~budget_s."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    threads = threads or min(16, os.cpu_count() or 1)
    loras = [(b, a, O.BF16, c) for (b, a, r, c) in case["loras"]]
    fmt = O.E4M3FN if case["fmt"] == 0 else O.E5M2
    args = (case["w"], fmt, case["scale_mode"], case["scales"], loras)
    t0 = time.perf_counter()
    reps = 0
    while True:
        O.read_bf16(*args, threads=threads)
        reps += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return threads, reps, dt


def cpu_config(cases, threads):
    """The oracle over one step of a workload: every tensor once on `threads`
    host threads, and the first tensor on one thread (extrapolated to the
    step by algorithmic bytes). Returns the figures for the bench line."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O

    def run(c, th):
        loras = [(b, a, O.BF16, co) for (b, a, r, co) in c["loras"]]
        fmt = O.E4M3FN if c["fmt"] == 0 else O.E5M2
        O.read_bf16(c["w"], fmt, c["scale_mode"], c["scales"], loras, threads=th)

    step_bytes = sum(synth_bytes(c) for c in cases)
    t0 = time.perf_counter()
    for c in cases:
        run(c, threads)
    dt = time.perf_counter() - t0
    t0 = time.perf_counter()
    run(cases[0], 1)
    dt1 = (time.perf_counter() - t0) * step_bytes / synth_bytes(cases[0])
    return {"GBps": round(step_bytes / dt / 1e9, 3), "s_per_step": round(dt, 4), "threads": threads,
            "GBps_1_thread": round(step_bytes / dt1 / 1e9, 3), "s_per_step_1_thread": round(dt1, 3),
            "sample": f"every tensor of one step once on {threads} threads; one thread on the first tensor "
                      f"({cases[0]['rows']}x{cases[0]['cols']}), extrapolated to the step by algorithmic bytes"}


def workload_cases(name, synth):
    """The tensors one step materialises, as synth.tensor_case dicts."""
    if name == "layer":
        return [synth.tensor_case(1002, ROWS, COLS, synth.E4M3FN, synth.SCALE_ROW, loras=((RANK, 1.0),))]
    if name == "dequant":
        return [synth.tensor_case(1001, ROWS, COLS, synth.E4M3FN, synth.SCALE_TENSOR, loras=())]
    if name == "block":
        return [synth.tensor_case(1003 * 100 + k, r, c, synth.E4M3FN, synth.SCALE_ROW, loras=((RANK, 1.0),))
                for k, (_, r, c) in enumerate(synth.BLOCK_LINEARS)]
    if name == "mixed":
        out = []
        for k, (nm, r, c) in enumerate(synth.BLOCK_LINEARS):
            ffn = nm.startswith("ff.")
            out.append(synth.tensor_case(1005 * 100 + k, r, c, synth.E5M2 if ffn else synth.E4M3FN,
                                         synth.SCALE_ROW if ffn else synth.SCALE_TENSOR,
                                         loras=((32, 1.0), (128, 0.5))))
        out.append(synth.tensor_case(1005 * 100 + 20, 4096, 4104, synth.E4M3FN, synth.SCALE_TENSOR,
                                     loras=((32, 1.0), (128, 0.5))))
        out.append(synth.tensor_case(1005 * 100 + 21, 4104, 16384, synth.E5M2, synth.SCALE_ROW,
                                     loras=((32, 1.0), (128, 0.5))))
        return out
    raise SystemExit(f"unknown workload {name}")


WORKLOAD_TEXT = {
    "model": "whole model: 48 DiT blocks (12.9B params) of e4m3fn + row scales and a rank-64 LoRA, "
             "safetensors files -> resident bf16, open to device sync",
    "model22b": "whole model: 82 DiT blocks (22.0B params) of e4m3fn + row scales and a rank-64 LoRA, "
                "safetensors files -> resident bf16, open to device sync",
    "model-mixed": "whole model: 48 DiT blocks, e5m2 FFN (row scales) / e4m3fn attention (one scale), "
                   "LoRAs r32 x1.0 + r128 x0.5, plus 4096x4104 and 4104x16384, open to device sync",
    "layer": "fused FP8 dequant + rank-64 LoRA merge, one 4096x4096 DiT linear, e4m3fn, per-row scales, bf16 out",
    "dequant": "FP8 e4m3fn -> bf16 dequant, one 4096x4096 tensor, per-tensor scale",
    "block": "fused dequant + rank-64 LoRA, one DiT block (8 x 4096^2, 16384x4096, 4096x16384), per-row scales, one grouped call",
    "mixed": "DiT block with e5m2 FFN (row scales) / e4m3fn attention (tensor scale), LoRAs r32 a=1 + r128 a=0.5, plus 4096x4104 and 4104x16384",
}


def tensor_arrays(c):
    """Host arrays of one case in upload order: weight, [scales], (B, A) per LoRA."""
    arrs = [c["w"]] + ([c["scales"]] if c["scales"] is not None else [])
    for b, a, _, _ in c["loras"]:
        arrs += [b, a]
    return arrs


def build_instances(ctx, cases, hip, stream, rotate_bytes=ROTATE_BYTES):
    """Device copies of the workload, repeated until they span rotate_bytes.
    Returns (instances, allocations, count); an instance is the list of
    grouped-call descriptors of one copy."""
    inst_bytes = sum(sum(x.nbytes for x in tensor_arrays(c)) + c["rows"] * c["cols"] * 2 for c in cases)
    n_inst = max(2, -(-rotate_bytes // inst_bytes))
    insts, allocs, nbytes_of = [], [], {}
    for k in range(n_inst):
        descs = []
        for ci, c in enumerate(cases):
            ptrs = []
            for x in tensor_arrays(c):
                p = ctx.alloc(x.nbytes)
                allocs.append(p)
                nbytes_of[p] = x.nbytes
                if k == 0:
                    ctx.upload(x, p)
                ptrs.append(p)
            if k > 0:
                for dst, sp, x in zip(ptrs, insts[0][ci]["_ptrs"], tensor_arrays(c)):
                    hip.copy_d2d(dst, sp, x.nbytes, stream)
            out = ctx.alloc(c["rows"] * c["cols"] * 2)
            allocs.append(out)
            nbytes_of[out] = c["rows"] * c["cols"] * 2
            q = 1 if c["scales"] is not None else 0
            loras = [(ptrs[1 + q + 2 * l], ptrs[2 + q + 2 * l], r, co) for l, (_, _, r, co) in enumerate(c["loras"])]
            for b_p, a_p, r, _ in loras:
                assert nbytes_of[b_p] == c["rows"] * r * 2 and nbytes_of[a_p] == r * c["cols"] * 2
            descs.append({"w": ptrs[0], "scales": ptrs[1] if q else None, "out": out, "rows": c["rows"],
                          "cols": c["cols"], "fmt": c["fmt"], "scale_mode": c["scale_mode"], "loras": loras,
                          "_ptrs": ptrs})
        insts.append(descs)
    return insts, allocs, n_inst


MODEL_WORKLOADS = {
    # name: (blocks, file variant, [(rank, strength)], seed)
    "model": (48, 0, [(64, 1.0)], 1004),
    "model22b": (82, 0, [(64, 1.0)], 1004),
    "model-mixed": (48, 1, [(32, 1.0), (128, 0.5)], 1005),
}


def model_dir(need_bytes, prefer=("/dev/shm", "/tmp")):
    """The first of `prefer` with room for the files."""
    for d in prefer:
        try:
            st = os.statvfs(d)
        except OSError:
            continue
        if st.f_bavail * st.f_frsize > need_bytes * 1.1:
            return d
    raise SystemExit(f"no directory with {need_bytes / 1e9:.1f} GB free for the model files")


def fs_type(path):
    """File-system type of the mount holding `path` (from /proc/mounts)."""
    best, typ = "", "unknown"
    try:
        with open("/proc/mounts") as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 3 and path.startswith(parts[1]) and len(parts[1]) >= len(best):
                    best, typ = parts[1], parts[2]
    except OSError:
        pass
    return typ


def drop_page_cache(paths):
    """Write back and evict the files' pages (posix_fadvise DONTNEED), so the
    next read of them comes from the storage device. Returns the fraction of
    their pages still resident afterwards (mincore), or None if unknown."""
    import mmap

    resident, total = 0, 0
    for p in paths:
        fd = os.open(p, os.O_RDONLY)
        try:
            os.fsync(fd)
            os.posix_fadvise(fd, 0, 0, os.POSIX_FADV_DONTNEED)
        finally:
            os.close(fd)
    try:
        libc = ctypes.CDLL(None, use_errno=True)
        libc.mincore.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        libc.mmap.restype = ctypes.c_void_p
        libc.mmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                              ctypes.c_long]
        libc.munmap.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
        page = mmap.PAGESIZE
        for p in paths:
            n = os.path.getsize(p)
            fd = os.open(p, os.O_RDONLY)
            try:
                addr = libc.mmap(None, n, mmap.PROT_READ, mmap.MAP_SHARED, fd, 0)
                if addr in (None, ctypes.c_void_p(-1).value):
                    return None
                try:
                    vec = (ctypes.c_ubyte * ((n + page - 1) // page))()
                    if libc.mincore(addr, n, vec) != 0:
                        return None
                    resident += sum(b & 1 for b in vec)
                    total += len(vec)
                finally:
                    libc.munmap(addr, n)
            finally:
                os.close(fd)
    except (OSError, AttributeError):
        return None
    return resident / total if total else 0.0


def run_model(name, reps, warmup, log_prefix="", host_threads=8, staging_mib=0, staging_slots=0, cold=False,
              check_tensors=12, mfma=False):
    """Whole-model materialisation: seeded FP8 checkpoint + LoRA files on
    disk, then per step: WeightStore.open (mmap, header parse, key rules) ->
    LoraFile.open + merge_lora -> materialize every linear into resident bf16
    -> device sync. Output buffers are allocated once, before the steps.
    cold: the files go to a disk-backed directory and their pages are evicted
    before every step, so `open` -> sync includes reading them from storage."""
    import ltx_weights as lw
    from ltx_weights import synth
    from ltx_weights.store import MAT_MFMA, KeyMap, LoraFile, WeightStore

    n_blocks, variant, loras, seed = MODEL_WORKLOADS[name]
    layout = synth.model_layout(n_blocks, variant)
    params = sum(r * c for _, _, _, r, c in layout)
    fp8_bytes = params
    scale_bytes = sum(4 * (r if sm == synth.SCALE_ROW else 1) for _, _, sm, r, _ in layout)
    factor_bytes = sum(2 * rk * (r + c) for _, _, _, r, c in layout for rk, _ in loras)
    h2d_bytes = fp8_bytes + scale_bytes + factor_bytes
    dev_bytes = sum(synth.algorithmic_bytes(r, c, sm, [rk for rk, _ in loras]) for _, _, sm, r, c in layout)
    d = model_dir(h2d_bytes, ("/tmp", "/var/tmp") if cold else ("/dev/shm", "/tmp"))
    if cold and fs_type(d) in ("tmpfs", "ramfs"):
        return {"skipped": f"no disk-backed directory with room ({d} is {fs_type(d)})"}
    mpath = os.path.join(d, f"ltxw_bench_{name}_{os.getpid()}.safetensors")
    lpaths = [os.path.join(d, f"ltxw_bench_{name}_{os.getpid()}_lora{k}.safetensors") for k in range(len(loras))]
    threads = min(16, os.cpu_count() or 1)
    res = {"blocks": n_blocks, "params": params, "h2d_bytes": h2d_bytes, "device_bytes": dev_bytes,
           "dir": d, "fs": fs_type(d)}
    try:
        t0 = time.perf_counter()
        synth.write_model(mpath, seed, n_blocks, variant, threads=threads)
        for k, (rk, _) in enumerate(loras):
            synth.write_lora(lpaths[k], seed + 1 + k, n_blocks, rk, variant, threads=threads)
        res["write_s"] = round(time.perf_counter() - t0, 3)
        log(f"{log_prefix}wrote {h2d_bytes / 1e9:.1f} GB of files to {d} ({res['fs']}) in {res['write_s']} s")

        keys = [k for k, *_ in layout]
        ctx = lw.Context(0, staging_bytes=staging_mib << 20, n_staging=staging_slots)
        ctx.set_host_threads(min(host_threads, threads))
        offs, total = [], 0
        for _, _, _, r, c in layout:
            offs.append(total)
            total += (2 * r * c + 255) // 256 * 256
        t0 = time.perf_counter()
        arena = ctx.alloc(total)
        res["alloc_s"] = round(time.perf_counter() - t0, 4)
        outs = [arena + o for o in offs]
        times, parts, resid = [], [], []
        last_store = None
        for it in range(warmup + reps):
            if cold:
                if last_store is not None:
                    last_store.close()
                    last_store = None
                resid.append(drop_page_cache([mpath] + lpaths))
            t0 = time.perf_counter()
            store = WeightStore.open([mpath], KeyMap.transformer())
            t1 = time.perf_counter()
            for k, (rk, strength) in enumerate(loras):
                lf = LoraFile.open(lpaths[k])
                store.merge_lora(lf, strength)
                lf.close()
            t2 = time.perf_counter()
            store.materialize(ctx, keys, outs, lw.OUT_BF16, MAT_MFMA if mfma else 0)
            t3 = time.perf_counter()
            ctx.synchronize()
            t4 = time.perf_counter()
            if it >= warmup:
                times.append(t4 - t0)
                parts.append((t1 - t0, t2 - t1, t3 - t2, t4 - t3))
            if last_store is not None:
                last_store.close()
            last_store = store
            log(f"{log_prefix}step {it}: {t4 - t0:.3f} s (open {t1 - t0:.3f}, merge {t2 - t1:.3f}, "
                f"host copies {t3 - t2:.3f}, drain {t4 - t3:.3f})")
        last_store.close()
        best = min(times)
        med = float(np.median(times))
        k = times.index(best)
        res.update({
            "s": round(med, 4), "s_best": round(best, 4), "steps": len(times),
            "s_open": round(parts[k][0], 4), "s_merge": round(parts[k][1], 4),
            "s_host_copies": round(parts[k][2], 4), "s_drain": round(parts[k][3], 4),
            "h2d_GBps": round(h2d_bytes / med / 1e9, 2), "device_GBps": round(dev_bytes / med / 1e9, 1),
            "page_cache": ("cold: pages evicted (fsync + posix_fadvise DONTNEED) before each step; "
                           f"resident fraction after eviction {resid[-1] if resid else None}")
            if cold else "warm (files written just before)",
        })

        # Parity on sampled rows of sampled tensors, inputs regenerated from the seeds.
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import gpu_util as U
        step_t = max(1, len(layout) // check_tensors)
        picks = sorted(set(list(range(0, len(layout), step_t)) + [len(layout) - 2, len(layout) - 1]))
        worst, over, cond = 0, 0, 0
        for i in picks:
            key, fmt, sm, r, c = layout[i]
            rows = np.unique(np.array([0, r // 3, r - 1]))
            w, sc = synth.model_rows(seed, key, fmt, sm, rows, c, r)
            ls = []
            for kk, (rk, strength) in enumerate(loras):
                b, a = synth.lora_factors_rows(seed + 1 + kk, key, rk, rows, r, c)
                ls.append((b, a, rk, strength))
            case = {"w": w, "scales": sc[rows] if sm == synth.SCALE_ROW else sc, "rows": len(rows), "cols": c,
                    "fmt": fmt, "scale_mode": sm, "loras": ls}
            got = np.empty((len(rows), c), dtype=np.uint16)
            for q, o in enumerate(rows):
                ctx.download(outs[i] + 2 * int(o) * c, got[q])
            if not mfma:  # the reference's operation order: bit for bit
                if not np.array_equal(got, U.oracle_bf16(case)):
                    raise AssertionError(f"{key}: exact materialisation differs from the oracle")
                continue
            stats = U.compare_lora_bf16(case, got)
            worst = max(worst, stats["max_ulp"])
            over += stats["n_over_1ulp"]
            cond += stats.get("n_cond", 0)
        res["parity"] = ({"tensors_checked": len(picks), "of_tensors": len(layout), "rows_per_tensor": 3,
                          "bit_exact": True} if not mfma else
                         {"tensors_checked": len(picks), "of_tensors": len(layout), "rows_per_tensor": 3,
                          "max_ulp": worst, "n_over_1ulp": over, "n_cond": cond, "bar": PARITY_BAR})
        res["kernels"] = ("MFMA LoRA products (LTXW_MAT_MFMA)" if mfma else
                          "reference operation order (materialize's default), bit-identical")
        log(f"{log_prefix}parity ok on {len(picks)} sampled tensors, max {worst} ulp")
        ctx.free(arena)
        ctx.close()
    finally:
        for pth in [mpath] + lpaths:
            try:
                os.unlink(pth)
            except OSError:
                pass
    return res


def main_model(args):
    res = run_model(args.workload, args.steps, args.warmup, host_threads=args.host_threads,
                    staging_mib=args.staging_mib, staging_slots=args.staging_slots, cold=args.cold,
                    mfma=args.mfma_materialise)
    line = {
        "metric": METRIC,
        "value": res.get("s"),
        "unit": "s",
        "n_gpus": 1,
        "steps": res.get("steps"),
        "warmup": args.warmup,
        "ms_per_step": round(res["s"] * 1e3, 2) if "s" in res else None,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic seeded safetensors files (FP8 weights, f32 scales, bf16 LoRA factors)",
        "config": {"workload": WORKLOAD_TEXT[args.workload] + (" (cold page cache)" if args.cold else ""),
                   "name": args.workload},
        "materialise": res,
        "roofline": None,
        "cpu_baseline": None,
    }
    print(json.dumps(line), flush=True)


class Lead:
    """Large streaming-dequant launches queued on the compute stream just
    before each timed region (--lead-ms, 200 ms by default): the GPU runs
    them between the pre-timing synchronize and the first timed launch, so
    the timed launches start with the GPU in its loaded steady state (clocks
    and power management settle over tens of milliseconds of load) and,
    under a profiler whose per-launch host cost exceeds the kernels' time,
    still run back to back. 2^30 FP8 elements of random non-NaN codes per
    launch (a 64 MiB random block repeated; about 0.55 ms each). Not part of
    any timed figure except the streaming ceiling, which times these
    launches themselves. Measured on one machine (us per step): one layer over
    200 steps 11.54-11.57 behind 200 ms of lead, 11.75 behind 10 ms, against
    11.50-11.52 over 2000 steps; the mixed block 257.7-257.9 behind 200 ms,
    258.2-258.7 over 800 steps without a lead, 264 over 200 steps without."""

    N = 1 << 30
    LAUNCH_US = 550.0

    def __init__(self, ctx):
        import ltx_weights as lw

        self.lw, self.ctx = lw, ctx
        self.w = ctx.alloc(self.N)
        self.out = ctx.alloc(2 * self.N)
        self.s = ctx.alloc(4)
        rng = np.random.default_rng(7)
        block = 1 << 26
        codes = rng.integers(0, 0x7F, size=block, dtype=np.uint8)  # 0x7F / 0xFF are the NaNs
        codes |= rng.integers(0, 2, size=block, dtype=np.uint8) << 7
        for off in range(0, self.N, block):
            ctx.upload(codes, self.w + off)
        ctx.upload(np.array([0.5], np.float32), self.s)

    def launch(self, n):
        for _ in range(n):
            self.ctx.dequant(self.w, self.N >> 14, 1 << 14, self.lw.FMT_E4M3FN, self.lw.SCALE_TENSOR, self.s, self.out)

    def queue(self, us):
        """Launches that keep the GPU busy for about `us` microseconds
        (LAUNCH_US each)."""
        self.launch(int(us / self.LAUNCH_US) + 1)

    def calibration_copies(self, hip, stream, n=4):
        """n device-to-device copies of 256 MiB (the first half of the output
        buffer into the second): the known-size dispatches that the HBM
        counters of a profiled run are scaled by."""
        size = 1 << 28
        for _ in range(n):
            hip.copy_d2d(self.out + size, self.out, size, stream)

    def free(self):
        for p in (self.w, self.out, self.s):
            self.ctx.free(p)


def stream_ceiling(ctx, hip, stream, lead, reps=20, lead_us=0.0):
    """The library's streaming dequant (16 FP8 bytes in, 32 bytes of bf16 out
    per thread) over 2^30 elements: the 1 B in / 2 B out pattern with no tile
    structure, the ceiling the fused kernels' traffic is compared with. `reps`
    launches timed back to back behind a queued lead."""
    lead.queue(max(reps * 20.0, lead_us))
    e0, e1 = hip.event(), hip.event()
    hip.record(e0, stream)
    lead.launch(reps)
    hip.record(e1, stream)
    us = hip.elapsed_ms(e0, e1) * 1e3 / reps
    gbps = (3.0 * Lead.N + 4) / (us * 1e-6) / 1e9
    return {"kernel": "k_dequant (ltxw_dequant, 2^30 e4m3fn codes, a 64 MiB random block repeated, one scale, bf16 out)",
            "us": round(us, 2), "GBps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4), "launches": reps}


def kernel_config(name, ctx, hip, stream, lead, steps, warmup, exact=False, check_rows=64, lead_us=0.0):
    """Times `steps` launches of one workload (after `warmup`), checks the
    last instance written against the oracle on sampled rows, and returns
    the figures of that workload."""
    import ltx_weights as lw
    from ltx_weights import synth

    log(f"[{name}] generating inputs")
    cases = workload_cases(name, synth)
    step_bytes = sum(synth.algorithmic_bytes(c["rows"], c["cols"], c["scale_mode"], [l[2] for l in c["loras"]])
                     for c in cases)
    flops = sum(synth.lora_flops(c["rows"], c["cols"], [l[2] for l in c["loras"]]) for c in cases)
    insts, allocs, n_inst = build_instances(ctx, cases, hip, stream)
    try:
        if exact:
            for inst in insts:
                for d in inst:
                    d["flags"] = lw.DESC_EXACT
        ctx.synchronize()
        descs = [ctx.make_descs(inst) for inst in insts]
        for k in range(warmup):
            ctx.grouped(descs[k % n_inst])
        ctx.synchronize()
        # Pre-heat (see Lead), then the timed launches queue up behind it.
        if lead_us > 0:
            lead.queue(lead_us)
        t_start, t_end = hip.event(), hip.event()
        hip.record(t_start, stream)
        h0 = time.perf_counter()
        for k in range(steps):
            ctx.grouped(descs[(warmup + k) % n_inst])
        host_s = time.perf_counter() - h0
        hip.record(t_end, stream)
        ms = hip.elapsed_ms(t_start, t_end)
        ctx.synchronize()
        us = ms * 1e3 / steps
        gbps = step_bytes / (us * 1e-6) / 1e9
        log(f"[{name}] {us:.2f} us/step, {gbps:.0f} GB/s ({gbps / HBM_PEAK_GBPS:.1%} of 8 TB/s); "
            f"host submission {host_s / steps * 1e6:.2f} us/step")

        # Parity of the last instance written, sampled rows of every tensor.
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import gpu_util as U
        last = insts[(warmup + steps - 1) % n_inst]
        par = {"tensors": len(cases), "rows_per_tensor": 0}
        worst, over, cond, frob = 0, 0, 0, 0.0
        for c, d in zip(cases, last):
            out = np.empty((c["rows"], c["cols"]), dtype=np.uint16)
            ctx.download(d["out"], out)
            sel = np.unique(np.linspace(0, c["rows"] - 1, check_rows).astype(np.int64))
            par["rows_per_tensor"] = len(sel)
            if c["loras"] and exact:
                if not np.array_equal(U.oracle_bf16(c, row_sel=sel), out[sel]):
                    raise AssertionError(f"[{name}] exact-mode output differs from the oracle")
                par["bit_exact"] = True
            elif c["loras"]:
                st = U.compare_lora_bf16(c, out[sel], row_sel=sel, label=f"bench {name}")
                worst = max(worst, st["max_ulp"])
                over += st["n_over_1ulp"]
                cond += st.get("n_cond", 0)
                frob = max(frob, st["frob_vs_rne_f64"])
            else:
                if not np.array_equal(U.oracle_bf16(c, row_sel=sel), out[sel]):
                    raise AssertionError(f"[{name}] dequant output differs from the oracle")
                par["bit_exact"] = True
        if any(c["loras"] for c in cases) and not exact:
            par.update({"max_ulp": worst, "n_over_1ulp": over, "n_cond": cond, "frob_vs_rne_f64_max": frob,
                        "bar": PARITY_BAR})
        log(f"[{name}] parity on sampled rows: {par}")
        traffic = read_traffic(name)
        return {"workload": WORKLOAD_TEXT[name] + (" (exact mode)" if exact else ""),
                "tensors": len(cases), "params": int(sum(c["rows"] * c["cols"] for c in cases)),
                "steps": steps, "warmup": warmup, "rotating_instances": n_inst,
                "us": round(us, 3), "GBps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "algorithmic_bytes": step_bytes, "lora_flops": flops,
                "traffic": traffic, "traffic_over_algorithmic": round(traffic / step_bytes, 4) if traffic else None,
                "host_submit_us_per_step": round(host_s / steps * 1e6, 2), "lead_us": round(lead_us),
                "parity": par, "_cases": cases}
    finally:
        for p in allocs:
            ctx.free(p)


CONFIG_OF = {"dequant": "1", "layer": "2", "block": "3", "mixed": "5"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--lead-ms", type=float, default=200.0,
                    help="ms of streaming-dequant launches queued ahead of each timed region (the GPU's loaded steady "
                         "state at the first timed launch; back-to-back launches under a profiler); 0 for none")
    ap.add_argument("--workload", default="layer", choices=sorted(WORKLOAD_TEXT))
    ap.add_argument("--configs", default="auto",
                    help="comma-separated kernel workloads measured beside the headline one "
                         "(auto: dequant,block,mixed beside the default layer workload; none: only the headline)")
    ap.add_argument("--config-steps", type=int, default=0,
                    help="timed launches per extra kernel workload (0: max(--steps, 20))")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline time budget (0 skips it)")
    ap.add_argument("--e2e", default="auto",
                    help="comma-separated whole-model runs beside the kernel workloads: model22b, model, "
                         "model-mixed, with -mfma (MFMA kernels) and/or -cold suffixes (auto: model22b, "
                         "model22b-mfma, model, model-mixed, model22b-cold beside the default layer workload; none)")
    ap.add_argument("--e2e-steps", type=int, default=3)
    ap.add_argument("--cold", action="store_true", help="whole-model workloads: evict the files' pages first")
    ap.add_argument("--host-threads", type=int, default=8,
                    help="host threads filling the pinned staging block in whole-model runs")
    ap.add_argument("--staging-mib", type=int, default=0,
                    help="pinned staging slot size in MiB for whole-model runs (0: the library default, 64)")
    ap.add_argument("--staging-slots", type=int, default=0,
                    help="pinned staging slots for whole-model runs (0: the library default, 16)")
    ap.add_argument("--mfma-materialise", action="store_true",
                    help="whole-model runs: LoRA deltas on the MFMA kernels (LTXW_MAT_MFMA) instead of "
                         "materialize's default reference order")
    ap.add_argument("--exact", action="store_true",
                    help="LoRA deltas in the reference's operation order (LTXW_DESC_EXACT, bit-identical)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the weight set shards by tensor with no exchange between GPUs).", file=sys.stderr)
        sys.exit(2)

    if args.workload in MODEL_WORKLOADS:
        return main_model(args)
    default_run = args.workload == "layer" and not args.exact
    if args.configs == "auto":
        extra = ["dequant", "block", "mixed"] if default_run else []
    elif args.configs == "none":
        extra = []
    else:
        extra = [c for c in args.configs.split(",") if c and c != args.workload]
    if args.e2e == "auto":
        e2e_runs = ["model22b", "model22b-mfma", "model", "model-mixed", "model22b-cold"] if default_run else []
    elif args.e2e == "none":
        e2e_runs = []
    else:
        e2e_runs = [x for x in args.e2e.split(",") if x]

    import ltx_weights as lw

    hip = Hip()
    ctx = lw.Context(0)
    stream = ctx.stream()
    lead = Lead(ctx)
    head = kernel_config(args.workload, ctx, hip, stream, lead, args.steps, args.warmup, exact=args.exact,
                         lead_us=args.lead_ms * 1e3)
    cases = head.pop("_cases")
    value = head["GBps"]
    configs = {CONFIG_OF.get(args.workload, args.workload): dict(head, name=args.workload)}
    csteps = args.config_steps or max(args.steps, 20)
    config_cases = {}
    for name in extra:
        r = kernel_config(name, ctx, hip, stream, lead, csteps, min(args.warmup, 5) or 1, lead_us=args.lead_ms * 1e3)
        config_cases[name] = r.pop("_cases")
        configs[CONFIG_OF.get(name, name)] = dict(r, name=name)
    ceiling = stream_ceiling(ctx, hip, stream, lead, lead_us=args.lead_ms * 1e3) if default_run else None
    if ceiling:
        log(f"streaming dequant ceiling {ceiling['GBps']:.0f} GB/s")
    lead.calibration_copies(hip, stream)
    ctx.synchronize()
    lead.free()
    ctx.close()

    cpu = None
    if args.cpu_seconds > 0:
        log("cpu baseline")
        threads, reps, dt = cpu_baseline(cases[0], args.cpu_seconds)
        c0 = cases[0]
        b0 = synth_bytes(c0)
        try:
            affinity = len(os.sched_getaffinity(0))
        except AttributeError:
            affinity = None
        cpu = {"value": round(b0 * reps / dt / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{reps} x the {c0['rows']}x{c0['cols']} tensor through the C oracle "
                         f"(reference operation order), {threads} threads, {dt:.1f} s",
               "s_per_tensor": round(dt / reps, 4), "host_cpus": os.cpu_count(), "host_cpus_usable": affinity}
        # One thread, as the reference runs (a scalar loop on one thread).
        _, reps1, dt1 = cpu_baseline(c0, min(5.0, args.cpu_seconds / 2), threads=1)
        cpu["value_1_thread"] = round(b0 * reps1 / dt1 / 1e9, 3)
        cpu["s_per_tensor_1_thread"] = round(dt1 / reps1, 4)
        # The other kernel workloads, one step each (reported beside their GPU figures).
        for name, cc in config_cases.items():
            log(f"cpu baseline: {name}")
            k = CONFIG_OF.get(name, name)
            configs[k]["cpu"] = cpu_config(cc, threads)
            configs[k]["gpu_over_cpu"] = round(configs[k]["GBps"] / configs[k]["cpu"]["GBps"], 1)

    e2e = {}
    for run in e2e_runs:
        name, cold, mfma = run, False, False
        if name.endswith("-cold"):
            name, cold = name[:-5], True
        if name.endswith("-mfma"):
            name, mfma = name[:-5], True
        log(f"whole-model materialisation ({run})")
        try:
            r = run_model(name, args.e2e_steps if not cold else 2, 1 if not cold else 0, log_prefix="  ",
                          host_threads=args.host_threads, staging_mib=args.staging_mib,
                          staging_slots=args.staging_slots, cold=cold, mfma=mfma)
            if cpu is not None and "device_bytes" in r:
                # The oracle's rate on this host applied to the model's device bytes.
                r["cpu_estimate_s"] = round(r["device_bytes"] / (cpu["value"] * 1e9), 1)
        except Exception as ex:  # reported in the line, never hides the kernel result
            r = {"error": f"{type(ex).__name__}: {ex}"}
        e2e[run] = dict(r, workload=WORKLOAD_TEXT[name] + (" (cold page cache)" if cold else "") +
                        (" (MFMA kernels)" if mfma else ""))

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1e3, 6),
        "host_submit_us_per_step": head["host_submit_us_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded: uniform non-NaN FP8 codes, U[1e-3,1e-1] scales, N(0,0.02^2) bf16 factors)",
        "config": {"workload": head["workload"], "name": args.workload + ("-exact" if args.exact else ""),
                   "tensors": head["tensors"], "params": head["params"],
                   "rotating_instances": head["rotating_instances"]},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": head["frac"], "traffic": head["traffic"],
                     "algorithmic_bytes": head["algorithmic_bytes"], "lora_flops": head["lora_flops"],
                     "stream_ceiling": ceiling,
                     "frac_of_stream_ceiling": round(value / ceiling["GBps"], 4) if ceiling else None},
        "parity": head["parity"],
        "configs": configs,
        "cpu_baseline": cpu,
        "materialise": e2e or None,
    }
    print(json.dumps(line), flush=True)


def synth_bytes(c):
    from ltx_weights import synth

    return synth.algorithmic_bytes(c["rows"], c["cols"], c["scale_mode"], [l[2] for l in c["loras"]])


if __name__ == "__main__":
    main()
