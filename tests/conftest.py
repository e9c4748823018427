import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "war-chest-bot-9000-_amd")
ORACLE = os.path.join(ROOT, "oracle")
for p in (PKG, ORACLE, os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

# Waves the service packs from jobs validated at submit are not checked on the
# host (unless WC_DEEP_CHECK=1): their uploads check them on the device, which
# is what the service tests run.


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X")

