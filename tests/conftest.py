"""Test configuration.

* registers the `gpu` marker (tests that need an MI355X and the HIP library);
* puts the package directory and the repository root on sys.path so that
  `import orthocache_gpu` resolves to orthocache-gpu_amd/orthocache_gpu and
  `import oracle` to the CPU checker;
* enables CPU flush-to-zero like the reference suite (tests/conftest.py:20-25
  of the reference).
"""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "orthocache-gpu_amd")
for p in (PKG_DIR, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built HIP library")
    try:
        import torch
        torch.set_flush_denormal(True)
    except Exception:
        pass


def pytest_terminal_summary(terminalreporter, exitstatus, config):
    """The achieved output errors of the GPU parity checks (tests/bars.py)."""
    try:
        from tests import bars
    except Exception:
        return
    for line in bars.summary_lines():
        terminalreporter.write_line(line)
