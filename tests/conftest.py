import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # PyTorch-ROCm wheels carry their own HIP runtime. Loaded after the one
    # libindecis_hip.so links (/opt/rocm), torch's finds no GPU ("No HIP GPUs
    # are available"); loaded first, the library shares it. Tests that hand
    # torch's device memory to the library then pass in any order.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
