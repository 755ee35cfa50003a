"""Whole-model materialisation at full size: a 48-block synthetic DiT
checkpoint (FP8 weights + f32 scales, 12.9 B parameters) and its LoRA
adapters written as safetensors files, memory-mapped and streamed through
WeightStore.open -> merge_lora -> materialize into resident bf16, every
tensor then checked on sampled rows against the oracle. This is the caller
loop of ltx-dit's loader, which reads every linear of every block
(crates/ltx-dit/src/load.rs:92-97,149-170), done as one materialize call.

Inputs of the oracle come from the same files (memory-mapped, only the
sampled rows and the A factors are read), so the check covers the staging
pipeline, the key rules and the merge bookkeeping as well as the kernels.
Bar: materialize's default (the reference's operation order) bit-identical
to the oracle on every tensor; with MAT_MFMA, gpu_util.compare_lora_bf16 on
every tensor (1 bf16 ulp of the reference's result, or no farther from the
exact value than the reference's own f32, or for an ill-conditioned element
the f32 forward-error bound; Frobenius <= 1e-3).
"""
import os
import sys
import time

import numpy as np
import pytest

import gpu_util as U
import ltx_weights as lw
import st_io
from ltx_weights import synth
from ltx_weights.store import MAT_MFMA, KeyMap, LoraFile, WeightStore

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def model_dir(need_bytes):
    for d in ("/dev/shm", "/tmp"):
        try:
            st = os.statvfs(d)
        except OSError:
            continue
        if st.f_bavail * st.f_frsize > need_bytes * 1.2:
            return d
    pytest.skip(f"no directory with {need_bytes / 1e9:.1f} GB free for the model files")


# (blocks, file variant, [(rank, strength)], seed)
SETS = {
    # 48 blocks of one DiT block's shapes, e4m3fn with per-row scales, one rank-64 LoRA.
    "48 blocks, rank 64": (48, 0, [(64, 1.0)], 4004),
    # The same 48 blocks with e5m2 FFN (row scales) and e4m3fn attention (one
    # scale), LoRAs r32 x1.0 then r128 x0.5, plus 4096x4104 and 4104x16384.
    "48 blocks mixed, r32 + r128, edge shapes": (48, 1, [(32, 1.0), (128, 0.5)], 4005),
}


# materialize's default (the reference's operation order: bit-identical) on
# both sets, and the MFMA kernels (MAT_MFMA: the tolerance) on the mixed one.
@pytest.mark.parametrize("name,mfma", [(n, False) for n in SETS] + [(list(SETS)[1], True)])
def test_whole_model_materialise_every_tensor(name, mfma):
    n_blocks, variant, loras, seed = SETS[name]
    name = name + (", MFMA kernels" if mfma else ", reference order")
    layout = synth.model_layout(n_blocks, variant)
    params = sum(r * c for _, _, _, r, c in layout)
    need = params + sum(2 * rk * (r + c) for _, _, _, r, c in layout for rk, _ in loras)
    d = model_dir(need)
    pid = os.getpid()
    mpath = os.path.join(d, f"ltxw_test_model_{pid}.safetensors")
    lpaths = [os.path.join(d, f"ltxw_test_model_{pid}_lora{k}.safetensors") for k in range(len(loras))]
    threads = min(16, os.cpu_count() or 1)
    ctx = None
    arena = None
    try:
        t0 = time.time()
        log(f"case: {name}: writing {need / 1e9:.1f} GB of files to {d}")
        synth.write_model(mpath, seed, n_blocks, variant, threads=threads)
        for k, (rk, _) in enumerate(loras):
            synth.write_lora(lpaths[k], seed + 1 + k, n_blocks, rk, variant, threads=threads)
        log(f"  written in {time.time() - t0:.1f} s; materialising {len(layout)} tensors ({params / 1e9:.2f} B params)")
        ctx = lw.Context(0)
        store = WeightStore.open([mpath], KeyMap.transformer())
        for k, (_, strength) in enumerate(loras):
            lf = LoraFile.open(lpaths[k])
            rep = store.merge_lora(lf, strength)
            lf.close()
            assert len(rep.matched_keys) == len(layout) and not rep.unmatched_lora_keys
        keys = [k for k, *_ in layout]
        offs, total = [], 0
        for _, _, _, r, c in layout:
            offs.append(total)
            total += (2 * r * c + 255) // 256 * 256
        arena = ctx.alloc(total)
        t1 = time.time()
        store.materialize(ctx, keys, [arena + o for o in offs], lw.OUT_BF16, MAT_MFMA if mfma else 0)
        ctx.synchronize()
        log(f"  materialised in {time.time() - t1:.3f} s; checking sampled rows of every tensor")
        mfile = st_io.open_mmap(mpath)
        lfiles = [st_io.open_mmap(p) for p in lpaths]
        worst, over = 0, 0
        for i, (key, fmt, sm, r, c) in enumerate(layout):
            rows = np.unique(np.array([(i * 7919) % r, r // 2, r - 1], dtype=np.int64))
            full = synth.CKPT_PREFIX + key
            w = np.asarray(mfile[full][2]).reshape(r, c)[rows]
            sc_all = np.asarray(mfile[full + "_scale"][2], dtype=np.float32)
            case_loras = []
            prefix = key[: -len(".weight")]  # adapters name the store keys
            for (rk, strength), lf in zip(loras, lfiles):
                b = np.asarray(lf[prefix + ".lora_B.weight"][2]).reshape(r, rk)[rows]
                a = np.asarray(lf[prefix + ".lora_A.weight"][2]).reshape(rk, c)
                case_loras.append((b, a, rk, strength))  # alpha absent: coeff = strength
            case = {"w": np.ascontiguousarray(w), "scales": sc_all[rows] if sm == synth.SCALE_ROW else sc_all[:1],
                    "rows": len(rows), "cols": c, "fmt": fmt, "scale_mode": sm, "loras": case_loras,
                    "label": f"{name}: {key}"}
            got = np.empty((len(rows), c), dtype=np.uint16)
            for q, o in enumerate(rows):
                ctx.download(arena + offs[i] + 2 * int(o) * c, got[q])
            if not mfma:
                assert np.array_equal(got, U.oracle_bf16(case)), f"{key}: differs from the reference order"
                continue
            stats = U.compare_lora_bf16(case, got)
            worst = max(worst, stats["max_ulp"])
            over += stats["n_over_1ulp"]
            if i % 60 == 0 or i == len(layout) - 1:
                log(f"  {i + 1}/{len(layout)} tensors checked, max {worst} ulp, {over} beyond 1 ulp")
        log(f"case: {name}: every tensor within the bar (max {worst} ulp, {over} elements beyond 1 ulp)"
            if mfma else f"case: {name}: every tensor bit-identical to the reference order")
    finally:
        if arena is not None:
            ctx.free(arena)
        if ctx is not None:
            ctx.close()
        for p in [mpath] + lpaths:
            try:
                os.unlink(p)
            except OSError:
                pass
