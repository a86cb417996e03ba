import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "qwen3-tts.cpp_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)

# The parity tests compare the device with the oracle bit for bit, so they
# run F16 prefills on the exact f64-MFMA GEMMs; the tests of the default fast
# form (fp16 MFMA, fp32 accumulation; a tolerance) switch it back on.
os.environ.setdefault("Q3T_PF_EXACT", "1")
# Likewise the multi-stream decode of F16 layers runs on the exact f64-MFMA
# GEMMs; the test of its default fp16-MFMA form switches that back.
os.environ.setdefault("Q3T_MS_EXACT", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the device C ABI")
    config.addinivalue_line("markers", "slow: full 0.6B-shape case")


@pytest.fixture(scope="session")
def oracle_lib():
    import q3t_oracle
    return q3t_oracle
