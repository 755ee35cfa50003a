"""The bf16 tolerance of the fused-path parity tests, exercised on the CPU:
it must accept the oracle's own output, reject a 2-ulp error in a
well-conditioned element, and admit a deviation in an ill-conditioned
element only within the f32 forward-error bound."""
import numpy as np
import pytest

import gpu_util as U
import ltx_weights as lw
from ltx_weights import synth


def bf16(x):
    return synth.bf16_from_f64(np.asarray(x, dtype=np.float64))


def cancel_case():
    """Element (0, 0) is -1 + 1*1 + 2^-15*2^-15 = 2^-30 (S = 2 + 2^-30); every
    other element is well conditioned."""
    rng = np.random.default_rng(3)
    rows, cols, rank = 4, 16, 2
    base = rng.normal(0.0, 0.5, size=(rows, cols))
    b = rng.normal(0.0, 0.1, size=(rows, rank))
    a = rng.normal(0.0, 0.1, size=(rank, cols))
    base[0, 0] = -1.0
    b[0] = [1.0, 2.0 ** -15]
    a[:, 0] = [1.0, 2.0 ** -15]
    return {"w": bf16(base), "scales": None, "rows": rows, "cols": cols, "fmt": lw.FMT_BF16,
            "scale_mode": lw.SCALE_NONE, "loras": [(bf16(b), bf16(a), rank, 1.0)]}


def test_accepts_oracle_output():
    case = cancel_case()
    st = U.compare_lora_bf16(case, U.oracle_bf16(case))
    assert st["n_over_1ulp"] == 0


def test_rejects_two_ulp_in_well_conditioned_element():
    case = cancel_case()
    got = U.oracle_bf16(case).copy()
    got[2, 5] += 2  # two steps away from the reference's own result
    with pytest.raises(AssertionError):
        U.compare_lora_bf16(case, got)


def test_ill_conditioned_element_within_bound():
    case = cancel_case()
    ref = U.oracle_bf16(case)
    assert U.bf16_to_f64(ref[:1, :1])[0, 0] == 2.0 ** -30  # the f32 chain is exact here
    got = ref.copy()
    got[0, 0] = 0  # |err| = 2^-30 <= (2 + 4) 2^-24 (2 + 2^-30)
    st = U.compare_lora_bf16(case, got)
    assert st["n_cond"] == 1 and st["cond_err_over_limit"] < 2e-3


def test_ill_conditioned_element_outside_bound():
    case = cancel_case()
    got = U.oracle_bf16(case).copy()
    got[0, 0] = bf16([2.0 ** -19])[0]  # |err| ~ 2^-19 > 6 * 2^-24 * 2 = 2^-20.4
    with pytest.raises(AssertionError):
        U.compare_lora_bf16(case, got)
