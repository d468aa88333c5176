import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "solidattention-repro_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libsa_hip.so)")


@pytest.fixture(scope="session")
def oracle_lib():
    import oracle
    if not os.path.exists(oracle.LIB_PATH):
        oracle.build(reference=False)
    return oracle


@pytest.fixture(scope="session")
def ref_lib(oracle_lib):
    if not oracle_lib.ref_available():
        pytest.skip("oracle/_ref/libsa_ref.so not built (reference sources absent at build time)")
    return oracle_lib


@pytest.fixture(scope="session")
def hip():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import solidattention_amd as sa
    sa.lib()
    return sa
