"""The benchmark receipt end to end on the GPU: the correctness gate passes and every section of
the reference's receipt (benchmarks/tensorops.py:276-295) is present with sane timings."""

from __future__ import annotations

import json

import pytest

from benchmarks import tensorops

pytestmark = pytest.mark.gpu


def test_receipt(dev, tmp_path):
    out = tmp_path / "r.json"
    receipt = tensorops.main(["--shape", "256x512x258", "--iterations", "2", "--output", str(out)])
    assert json.loads(out.read_text()) == receipt
    gate = receipt["correctness"]
    assert gate["hipW4A4ExactIntegerDot"] is True
    assert gate["hipW4A4Fp6ExactIntegerDotAndSameOutput"] is True
    assert gate["hipW4A4Float32EpilogueMaximumAbsoluteError"] <= 1e-5
    assert gate["hipW4A16MaximumAbsoluteError"] <= gate["hipW4A16Tolerance"]
    (bench,) = receipt["benchmarks"]
    assert bench["shape"] == {"m": 256, "k": 512, "n": 258}
    sections = [bench["denseBf16"], *bench["activationPreparation"].values(), *bench["kernelOnly"].values(),
                *bench["completeLinearPath"].values()]
    assert len(sections) == 14  # the reference's 11, plus FP6 preparation, kernel and complete path
    assert {"hipW4A4Fp6"} <= set(bench["kernelOnly"]) and {"hipW4A4Fp6"} <= set(bench["completeLinearPath"])
    for s in sections:
        assert len(s["seconds"]) == 2 and 0 < s["bestSeconds"] <= s["medianSeconds"]
        assert s["totalPeakGiB"] > 0
    for s in (*bench["kernelOnly"].values(), *bench["completeLinearPath"].values()):
        assert s["speedupVsDenseBf16"] > 0
