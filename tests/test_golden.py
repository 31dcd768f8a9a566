"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) against the oracle as it is now: any change to
the oracle's arithmetic shows here, bit for bit.  Also the known answers the
fixtures carry from the reference's own tests."""
from pathlib import Path

import numpy as np
import pytest

import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"

import importlib.util  # noqa: E402

_spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_golden.py")
make_golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_golden)


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("group", sorted(make_golden.GROUPS))
def test_oracle_reproduces_its_fixtures_bit_for_bit(group):
    want = load(group)
    got = {k: np.asarray(v) for k, v in make_golden.GROUPS[group]().items()}
    assert sorted(got) == sorted(want)
    for k in want:
        np.testing.assert_array_equal(got[k], want[k], err_msg=f"{group}.{k}")


def test_fixture_known_answers():
    r = load("route")
    # ffn.rs:1128-1147: experts [7, 1, 4, 2], renormalised weights, ratio e
    np.testing.assert_array_equal(r["kat_experts"], [7, 1, 4, 2])
    w = r["kat_weights"]
    assert abs(float(w.sum()) - 1.0) < 1e-6
    assert abs(w[0] / w[1] - np.e) < 1e-5
    a = load("attend")
    np.testing.assert_array_equal(a["qwen1_out"], np.concatenate([a["qwen1_v"][h // 7 * 64:(h // 7 + 1) * 64]
                                                                  for h in range(14)]))
    s = load("small")
    assert abs(float(s["softmax"].sum()) - 1.0) < 1e-6
    q = load("quant")
    assert np.all(q["q8_qs"][32:64] == 0) and q["q8_scales"][1] == 0.0
