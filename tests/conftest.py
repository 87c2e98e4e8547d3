import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librocm_ribn on the device)")


def _built():
    return os.path.exists(os.path.join(ROOT, "ribn_amd", "librocm_ribn.so")) and os.path.exists(
        os.path.join(ROOT, "oracle", "liboracle.so"))


if not _built():   # build only when nothing is built yet
    import __graft_entry__
    __graft_entry__.build()
