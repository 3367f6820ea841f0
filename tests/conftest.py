import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
  sys.path.insert(0, ROOT)


def pytest_configure(config):
  config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(autouse=True)
def _gpu_guard(request):
  """A gpu-marked test never degrades to a skip or a host path: no GPU is a failure."""
  if request.node.get_closest_marker("gpu") is not None:
    import torch
    if not torch.cuda.is_available():
      pytest.fail("gpu test run without a visible GPU")
  yield


@pytest.fixture
def reset_runtime():
  from sparsefold_amd.runtime import config
  from sparsefold_amd import backends
  yield
  config.reset()
  config.configure_runtime(backend="torch")
  backends.init()
  config.reset()
