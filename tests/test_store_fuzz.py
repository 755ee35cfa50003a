"""Mutation fuzzing of the safetensors front end (no GPU).

`WeightStore.open` and `LoraFile.open` read untrusted files; whatever the
bytes, they must either open (and then answer keys / shape / dtype /
metadata queries consistently) or raise one of the library's errors. A crash
of the native parser ends this process, so surviving the loop is the check.
The mutations are seeded: byte flips and overwrites in the header, length
field changes, truncation and extension.
"""
import struct

import numpy as np
import pytest

import ltx_weights as lw
import st_io
from ltx_weights.store import LoraFile, WeightStore

ERRORS = (lw.WeightError,)


def base_file(path):
    rng = np.random.default_rng(3)
    tensors = [
        ("blk.0.attn.weight", "F8_E4M3", [4, 8], rng.integers(0, 120, 32).astype(np.uint8)),
        ("blk.0.attn.weight_scale", "F32", [4], rng.random(4).astype(np.float32)),
        ("blk.0.ff.weight", "BF16", [2, 3], rng.integers(0, 1 << 15, 6).astype(np.uint16)),
        ("blk.0.norm", "F32", [5], rng.random(5).astype(np.float32)),
        ("empty", "F16", [0, 3], np.zeros(0, dtype=np.uint16)),
    ]
    st_io.write(path, tensors, {"format": "pt", "note": "fuzz"})
    return path.read_bytes()


def lora_file(path):
    rng = np.random.default_rng(4)
    tensors = [
        ("blk.0.attn.lora_A.weight", "BF16", [2, 8], rng.integers(0, 1 << 15, 16).astype(np.uint16)),
        ("blk.0.attn.lora_B.weight", "BF16", [4, 2], rng.integers(0, 1 << 15, 8).astype(np.uint16)),
        ("blk.0.attn.alpha", "F32", [], np.array([2.0], dtype=np.float32)),
    ]
    st_io.write(path, tensors, {"ic_layout": "x"})
    return path.read_bytes()


def mutate(rng, blob):
    b = bytearray(blob)
    hlen = struct.unpack("<Q", bytes(b[:8]))[0]
    kind = rng.integers(0, 6)
    if kind == 0:  # flip bits in the header text
        for _ in range(int(rng.integers(1, 4))):
            i = 8 + int(rng.integers(0, hlen))
            b[i] ^= 1 << int(rng.integers(0, 8))
    elif kind == 1:  # overwrite header bytes with JSON-significant characters
        for _ in range(int(rng.integers(1, 4))):
            i = 8 + int(rng.integers(0, hlen))
            b[i] = ord(rng.choice(list('{}[],:"0123456789-.eE\\ ')))
    elif kind == 2:  # change the header length field
        n = max(0, hlen + int(rng.integers(-16, 17)))
        if rng.random() < 0.2:
            n = int(rng.integers(0, 1 << 40))
        b[:8] = struct.pack("<Q", n)
    elif kind == 3:  # truncate
        del b[int(rng.integers(0, len(b))):]
    elif kind == 4:  # extend the data section
        b += bytes(int(rng.integers(1, 64)))
    else:  # rewrite a digit inside the header (offsets and shapes)
        digits = [i for i in range(8, 8 + hlen) if chr(b[i]).isdigit()]
        if digits:
            b[digits[int(rng.integers(0, len(digits)))]] = ord(str(int(rng.integers(0, 10))))
    return bytes(b)


def exercise_store(s):
    for k in s.keys():
        assert s.contains(k)
        shape = s.shape(k)
        assert all(d >= 0 for d in shape)
        s.dtype(k)
    s.metadata("note")
    s.metadata("absent")


@pytest.mark.parametrize("seed", range(4))
def test_open_survives_mutated_files(tmp_path, seed):
    blob = base_file(tmp_path / "base.safetensors")
    rng = np.random.default_rng(1000 + seed)
    opened = failed = 0
    for k in range(400):
        p = tmp_path / f"m{k}.safetensors"
        p.write_bytes(mutate(rng, blob))
        try:
            s = WeightStore.open([p])
        except ERRORS:
            failed += 1
            continue
        try:
            exercise_store(s)
        finally:
            s.close()
        opened += 1
    assert opened + failed == 400
    assert failed > 0  # the mutations do reach the error paths


@pytest.mark.parametrize("seed", range(2))
def test_lora_open_survives_mutated_files(tmp_path, seed):
    blob = lora_file(tmp_path / "lora.safetensors")
    rng = np.random.default_rng(2000 + seed)
    for k in range(300):
        p = tmp_path / f"l{k}.safetensors"
        p.write_bytes(mutate(rng, blob))
        try:
            lf = LoraFile.open(p)
        except ERRORS:
            continue
        try:
            for name in lf.tensor_names():
                assert lf.tensor_info(name) is not None
            lf.metadata("ic_layout")
            try:
                lf.ic_layout()
            except ERRORS:
                pass
        finally:
            lf.close()


def test_parser_under_address_and_ub_sanitizers(tmp_path):
    """The header parser alone, built with -fsanitize=address,undefined,
    through 50k seeded mutations (tests/fuzz/fuzz_parse.cpp)."""
    import os
    import shutil
    import subprocess

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not available")
    here = os.path.dirname(os.path.abspath(__file__))
    csrc = os.path.join(os.path.dirname(here), "ltx-rust_amd", "csrc")
    exe = tmp_path / "fuzz_parse"
    build = subprocess.run([gxx, "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                            "-fno-omit-frame-pointer", "-I", csrc, "-o", str(exe),
                            os.path.join(here, "fuzz", "fuzz_parse.cpp"), os.path.join(csrc, "safetensors.cpp")],
                           capture_output=True, text=True)
    if build.returncode != 0 and "asan" in build.stderr.lower():
        pytest.skip("sanitizer runtime is not available: " + build.stderr[-200:])
    assert build.returncode == 0, build.stderr[-2000:]
    run = subprocess.run([str(exe), "50000"], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, (run.stdout + run.stderr)[-2000:]
    ok, bad = (int(x) for x in run.stdout.split()[1::2])
    assert ok + bad == 50000 and ok > 0 and bad > 0
