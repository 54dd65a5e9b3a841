import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


def gpu_available() -> bool:
    import torch
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


class _ReloadingEnviron(type(os.environ)):
    """os.environ whose MCQ4_* writes also re-read the library's switches.

    libmcq4.so reads its MCQ4_* test switches once (and again only on
    mcq4_reload_options), never per call; the tests flip them through
    os.environ / monkeypatch, so each such write reloads them here.
    """

    def _reload(self, key):
        if str(key).startswith("MCQ4_"):
            try:
                from metalops_amd import _lib
            except ImportError:        # library not built: nothing to reload
                return
            _lib.reload_options()

    def __setitem__(self, key, value):
        super().__setitem__(key, value)
        self._reload(key)

    def __delitem__(self, key):
        super().__delitem__(key)
        self._reload(key)


os.environ.__class__ = _ReloadingEnviron
