"""Pins the CPU oracle: reference golden vectors, reference known-answer
tests, an independent implementation (torch's FP8/bf16 casts), closed-form
invariants, and planted mistakes that each check must catch."""
import numpy as np
import pytest

import golden_checks as G
import oracle_lib as O


@pytest.mark.parametrize("check", G.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_check(check):
    ok, msg = check()
    assert ok, msg


def test_reference_fixture_files_match_committed_vectors():
    """When the reference tree is present, the committed vectors are its fixtures."""
    import json
    import os
    import st_io

    root = "/root/reference/crates/ltx-weights/tests/fixtures"
    if not os.path.isdir(root):
        pytest.skip("reference tree not present")
    with open(G.REF_FIXTURES) as f:
        committed = json.load(f)["files"]
    for stem, entry in committed.items():
        tensors, meta = st_io.read(os.path.join(root, stem + ".safetensors"))
        assert meta == entry["metadata"]
        for name, t in entry["tensors"].items():
            assert tensors[name][2].tobytes().hex() == t["hex"]


def test_decode_matches_torch_casts_all_codes():
    torch = pytest.importorskip("torch")
    codes = np.arange(256, dtype=np.uint8)
    for fmt, tdt in ((O.E4M3FN, torch.float8_e4m3fn), (O.E5M2, torch.float8_e5m2)):
        mine = O.decode(codes, fmt)
        theirs = torch.from_numpy(codes.copy()).view(tdt).float().numpy()
        nan_m, nan_t = np.isnan(mine), np.isnan(theirs)
        assert np.array_equal(nan_m, nan_t)
        assert np.array_equal(mine[~nan_m].view(np.uint32), theirs[~nan_t].view(np.uint32))
        # the reference's NaN is f32::NAN (0x7FC00000), positive quiet
        assert np.all(mine[nan_m].view(np.uint32) == 0x7FC00000)


def test_bf16_rne_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    u = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32)
    u[::7] = (u[::7] & 0xFFFF0000) | 0x8000          # exact ties
    u[1::7] = (u[1::7] & 0xFFFE0000) | 0x8000         # ties with even LSB
    u[2::7] = u[2::7] & 0x807FFFFF                    # subnormals
    x = u.view(np.float32)
    finite = np.isfinite(x) | np.isinf(x)
    mine = O.read_bf16(x.reshape(1, -1), O.F32).ravel()
    theirs = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(mine[finite], theirs[finite])
    # NaN: quiet bit set, sign and top payload kept (half 2.7.1 rule)
    nanx = u[~finite]
    assert np.array_equal(mine[~finite], ((nanx >> 16) | 0x40).astype(np.uint16))


def test_f16_widening_matches_torch_all_codes():
    """A second independent binary16 implementation (torch) on every
    non-NaN code; NaN codes as a class."""
    torch = pytest.importorskip("torch")
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    mine = O.decode(codes, O.F16)
    theirs = torch.from_numpy(codes.view(np.int16).copy()).view(torch.float16).float().numpy()
    nan_m, nan_t = np.isnan(mine), np.isnan(theirs)
    assert np.array_equal(nan_m, nan_t)
    assert np.array_equal(mine[~nan_m].view(np.uint32), theirs[~nan_t].view(np.uint32))


def test_f32_mt_is_bit_identical_to_single_thread():
    w, scales, loras = G.random_case(67, 96, 8, seed=11, nloras=2)
    one = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, scales, loras, threads=1)
    many = O.read_f32(w, O.E4M3FN, O.SCALE_ROW, scales, loras, threads=5)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))


# Every planted mistake must make at least one check fail.
@pytest.mark.parametrize("mut", range(1, 12))
def test_checks_catch_planted_mistake(mut):
    failed = []
    with O.mutation(mut):
        for check in G.ALL_CHECKS:
            ok, _ = check()
            if not ok:
                failed.append(check.__name__)
    assert failed, f"mutation {mut} passed every check"
