import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


# The CPU tests inspect the matrix-core path on small fixtures, below the
# size heuristics; the GPU tests set their own modes per module.
os.environ.setdefault("THVM_HIP_DENSE_FORCE", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
