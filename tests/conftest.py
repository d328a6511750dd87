import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "wgpu-ocr_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def rec_model_path():
    from ocrhip import synth
    return synth.model_path("rec")


@pytest.fixture(scope="session")
def det_model_path():
    from ocrhip import synth
    return synth.model_path("det")


@pytest.fixture(scope="session")
def rec_oracle(rec_model_path):
    from oracle import onnx_read
    return onnx_read.load(rec_model_path)


@pytest.fixture(scope="session")
def det_oracle(det_model_path):
    from oracle import onnx_read
    return onnx_read.load(det_model_path)


@pytest.fixture(scope="session")
def ctx():
    import ocrhip
    c = ocrhip.Context()
    yield c
    c.close()


@pytest.fixture(scope="session")
def recognizer(ctx, rec_model_path):
    import ocrhip
    return ocrhip.Recognizer(ctx, rec_model_path)


@pytest.fixture(scope="session")
def detector(ctx, det_model_path):
    import ocrhip
    return ocrhip.Detector(ctx, det_model_path)
