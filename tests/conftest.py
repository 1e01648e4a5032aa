"""Test configuration: import paths, the ``gpu`` marker and shared fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PACKAGE_DIR = ROOT / "radeon-kernels_amd"
for entry in (str(ROOT), str(PACKAGE_DIR)):
    if entry not in sys.path:
        sys.path.insert(0, entry)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run with -m gpu on the GPU host")


@pytest.fixture(scope="session")
def gpu():
    """The first visible gfx950 device, or skip."""

    import torch

    if not torch.cuda.is_available():
        pytest.skip("no visible ROCm GPU")
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":", 1)[0]
    if arch != "gfx950":
        pytest.skip(f"needs gfx950, found {arch}")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def palib(gpu):
    from radeon_kernels.cabi import library

    return library()


@pytest.fixture(scope="session")
def kvlib(gpu):
    from radeon_kernels.cabi import kv_library

    return kv_library()


@pytest.fixture(scope="session")
def c5_case(gpu):
    """The 128-sequence ragged workload drawn on the CPU (checked against its committed SHA-256
    digests), its float64 oracle over all 128 sequences, and a GPU copy of its inputs."""

    import json

    from _helpers import oracle64_rows, to_device
    from benchmarks.workloads import input_digests, make_inputs

    golden = json.loads((ROOT / "tests" / "golden" / "c5_inputs.json").read_text())
    data = make_inputs("c5")
    assert data["contexts"] == golden["contexts"] and data["num_blocks"] == golden["num_blocks"]
    assert input_digests(data) == golden["sha256"], "c5 inputs differ from the committed digests"
    sys.stderr.write("[case] c5 oracle over 128 sequences\n")
    sys.stderr.flush()
    expected = oracle64_rows(data)
    return {"cpu": data, "gpu": to_device(data, gpu), "expected": expected}
