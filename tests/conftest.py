import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


# GPU test files that have not yet passed on a GPU: collected after every other test (and before the
# no-allocation test, which is collected last), so that under `pytest -x` a first-run failure in one of them
# cannot hide the results of the tests that have run before. Remove a file from this set once it has passed.
FIRST_RUN = {
    "test_gpu_attention_addr.py", "test_gpu_cond.py", "test_gpu_configs.py", "test_gpu_dit_graph.py",
    "test_gpu_gemm_scales.py", "test_gpu_gemm_wahead.py", "test_gpu_reference_step.py",
}


def pytest_collection_modifyitems(config, items):
    def rank(item):
        name = os.path.basename(str(item.fspath))
        return 2 if name.startswith("test_zz") else 1 if name in FIRST_RUN else 0
    items[:] = sorted(items, key=rank)  # stable: the usual order within each group


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libkh.so on cuda:0)")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
