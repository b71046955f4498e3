import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(GOLDEN, "golden.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def golden_arrays():
    return dict(np.load(os.path.join(GOLDEN, "golden_arrays.npz")))


@pytest.fixture(scope="session")
def tiny_images(tmp_path_factory):
    """The fixture models written by this repository's writer (byte-identical with the
    reference writer, pinned by test_format.py): name -> path."""
    from trixium_amd import configs as C, synth, bons
    d = tmp_path_factory.mktemp("img")
    out = {}
    for cfg, seed, name, fp in ((C.TINY, 0, "tiny-qwen3", True), (C.TINY_HYBRID, 1, "tiny-hybrid", True),
                                (C.TINY, 3, "tiny-ternemb", False)):
        for t5 in (True, False):
            p = str(d / f"{name}-t{int(t5)}.img")
            bons.write_image(cfg, synth.small_model_tensors(cfg, seed, fp), 1, p, trit5=t5)
            out[(name, t5)] = p
    return out
