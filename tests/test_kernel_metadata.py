"""Code-object metadata of the built library's gfx950 kernels (CPU only).

No kernel may use private (scratch) memory or spill VGPRs: a kernel with
a private segment makes the HIP runtime provide scratch backing memory when it
is dispatched, which the allocation-free grouped call
(ltxw_dequant_lora_grouped_noalloc) promises never to need, and a spill costs
memory round trips inside the hot loops. The reference-order kernel is tuned
for five waves per SIMD (at most 96 VGPRs and no AGPRs); this pins that too.

The metadata is read from the library's own `.hip_fatbin` section with the
ROCm LLVM tools (llvm-objcopy, clang-offload-bundler, llvm-readelf); the test
is skipped where they are absent."""
import os
import shutil
import subprocess

import pytest
import yaml

from ltx_weights import _native

LLVM = "/opt/rocm/llvm/bin"
TOOLS = ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _kernels(tmp):
    lib = _native.LIB_PATH
    if not os.path.exists(lib):
        pytest.skip("libltxw.so is not built")
    if not all(os.path.exists(os.path.join(LLVM, t)) for t in TOOLS):
        pytest.skip("ROCm LLVM tools not installed")
    fat = os.path.join(tmp, "fatbin.bin")
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", lib, os.devnull],
                   check=True, capture_output=True)
    data = open(fat, "rb").read()
    offs = []
    at = data.find(MAGIC)
    while at >= 0:
        offs.append(at)
        at = data.find(MAGIC, at + 1)
    assert offs, "no offload bundle in .hip_fatbin"
    kernels = []
    for k, o in enumerate(offs):
        end = offs[k + 1] if k + 1 < len(offs) else len(data)
        bundle = os.path.join(tmp, f"b{k}.bin")
        co = os.path.join(tmp, f"b{k}.co")
        with open(bundle, "wb") as f:
            f.write(data[o:end])
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", f"--input={bundle}",
                        f"--targets={TARGET}", f"--output={co}"], check=True, capture_output=True)
        notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", co], check=True, capture_output=True,
                               text=True).stdout.splitlines()
        start = next(i for i, line in enumerate(notes) if line.strip() == "---")
        stop = next(i for i, line in enumerate(notes) if i > start and line.strip() == "...")
        meta = yaml.safe_load("\n".join(notes[start + 1:stop]))
        kernels += meta["amdhsa.kernels"]
    return kernels


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    return _kernels(str(tmp_path_factory.mktemp("codeobj")))


def test_no_kernel_uses_scratch_or_spills_vgprs(kernels):
    bad = [(k[".name"], k[".private_segment_fixed_size"], k[".vgpr_spill_count"])
           for k in kernels
           if k[".private_segment_fixed_size"] or k[".vgpr_spill_count"] or k.get(".uses_dynamic_stack", False)]
    assert not bad, bad


def one_round(name):
    """Fused kernels instantiated for one-round launches (their last template
    argument, WFIRST, is true: the mangled name ends in Lb1EE + JobTable)."""
    return "k_fused_pair" in name and name.endswith("Lb1EEEvNS_8JobTableE")


def test_sgpr_spills_bounded(kernels):
    """SGPR spills go to VGPR lanes (no memory), but each costs a lane write
    and a read on the issue path. A NaN test with one 64-bit ballot mask per
    value spilled some 350 SGPRs in every fused kernel; the probe form leaves
    only several-LoRA kernels of 4 K-steps and more spilling (their per-step
    factor pointers), about 100 at most at 7 K-steps. The one-round
    instantiations keep the ballots, which measured faster there."""
    rest = [k for k in kernels if not one_round(k[".name"])]
    worst = max(rest, key=lambda k: k[".sgpr_spill_count"])
    assert worst[".sgpr_spill_count"] <= 128, (worst[".name"], worst[".sgpr_spill_count"])
    single = [k for k in rest if "k_fused_pairIL" in k[".name"] or "k_dequant" in k[".name"] or "k_exact" in k[".name"]]
    assert single and all(k[".sgpr_spill_count"] == 0 for k in single), [
        (k[".name"], k[".sgpr_spill_count"]) for k in single if k[".sgpr_spill_count"]]
    assert any(one_round(k[".name"]) for k in kernels)


def test_expected_kernels_present(kernels):
    names = [k[".name"] for k in kernels]
    for stem in ("k_fill_words", "k_dequant_tile", "k_dequant", "k_generic", "k_exact", "k_fused_pair",
                 "k_fused_pair_multi"):
        assert any(stem in n for n in names), stem
    # Two output types x six factor types of the reference-order kernel.
    assert sum("k_exact" in n for n in names) == 12


def test_reference_order_kernel_fits_five_waves(kernels):
    ex = [k for k in kernels if "k_exact" in k[".name"]]
    assert ex
    for k in ex:
        assert k[".agpr_count"] == 0 and k[".vgpr_count"] <= 96, (k[".name"], k[".vgpr_count"], k[".agpr_count"])
