import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "ref: needs the reference leaf build under oracle/_ref")


def pytest_collection_modifyitems(config, items):
    from tests import helpers
    no_ref = not helpers.ref_available()
    for item in items:
        if no_ref and "ref" in item.keywords:
            item.add_marker(pytest.mark.skip(reason="oracle/_ref was not built (reference tree absent)"))
