"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need a visible HIP device and the built library
(diffuse-rs_amd/lib/libdr_attn.so); everything else runs on the CPU.
"""
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "diffuse-rs_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")
