"""pytest configuration: markers and import paths.

`gpu` marks tests that need an MI355X; the CPU suite runs with -m "not gpu".
The package directory tt-lang_amd/ (not an importable name itself) is put on
sys.path so `ttlhip`, `ttl`, `ttnn` resolve to this build's modules.
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "tt-lang_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU (gfx950)")
