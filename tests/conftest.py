import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for path in (REPO / "kimi-k3-pytorch_amd", REPO):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def pytest_collection_modifyitems(config, items):
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def segments():
    """Force the MFMA prefill's segment length for one test (the library's
    kda_set_segment_chunks: L >= 1 chunks per segment, 0 one segment per
    sequence), restoring the library's own plan afterwards."""
    from kda import _lib

    yield _lib.set_segment_chunks
    _lib.set_segment_chunks(-1)


def pytest_sessionfinish(session, exitstatus):
    # the measured errors of the full-size parity tests, when a record is asked for
    import json
    import os

    path = os.environ.get("KDA_PARITY_RECORD")
    if not path:
        return
    from tests._inputs import MARGINS

    Path(path).parent.mkdir(parents=True, exist_ok=True)
    Path(path).write_text(json.dumps(MARGINS, indent=1))
