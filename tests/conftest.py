"""pytest configuration: the ``gpu`` marker and import paths.

``-m "not gpu"`` runs on any host (oracle, host logic, library symbols);
``-m gpu`` needs a ROCm device and the built ``libnmce.so``.
"""

import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "nano-megatron_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built libnmce.so")
