"""The benchmark receipt's argument handling on the CPU (benchmarks/tensorops.py:298-330 of the
reference): shape parsing rules, iteration checks and refuse-to-overwrite, all before any
device work."""

from __future__ import annotations

import argparse

import pytest

from benchmarks import tensorops


def test_parse_shape():
    assert tensorops.parse_shape("1536x3072x21504") == (1536, 3072, 21504)
    for bad in ("1536x3000x64", "1x256x3", "0x256x2", "axbxc", "1x2"):
        with pytest.raises(argparse.ArgumentTypeError):
            tensorops.parse_shape(bad)


def test_refusals(tmp_path):
    out = tmp_path / "receipt.json"
    out.write_text("{}")
    with pytest.raises(FileExistsError, match="Refusing to overwrite"):
        tensorops.main(["--output", str(out)])
    with pytest.raises(ValueError, match="iterations"):
        tensorops.main(["--iterations", "0"])
