"""pytest configuration: the `gpu` marker and the repository root on sys.path."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")
    # registers the torch.ops.pragnosia namespace for every test module, whichever subset runs (the library itself
    # loads on the first call)
    import pragnosia_amd.ops  # noqa: F401
