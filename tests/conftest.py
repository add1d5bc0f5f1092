"""Test configuration: import paths and the `gpu` marker.

GPU tests (`-m gpu`) need a visible HIP device and the prebuilt
libmvme_paged.so; everything else runs on the CPU.
"""

from pathlib import Path
import sys

ROOT = Path(__file__).resolve().parents[1]
for path in (ROOT / "myvllm-mini-engine_amd", ROOT):
    if str(path) not in sys.path:
        sys.path.insert(0, str(path))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built HIP library")
