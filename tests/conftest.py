"""pytest configuration: import paths and the `gpu` marker.

`-m "not gpu"` runs on any host (oracle, codecs, host logic, library loading and
validation); `-m gpu` needs one MI355X (gfx950) and calls the HIP library through its C ABI.
"""
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
for sub in ("sixi-asi_amd", "oracle"):
    p = str(ROOT / sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs one MI355X (gfx950) GPU and the built HIP library")
