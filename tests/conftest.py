import math
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, ROOT)

# Sampled-row parity margins: every oracle.sample_token made by a GPU test is the expectation of a
# device row, so its cut margin |run - p| and draw margin |acc - r| are kept and summarised in
# one line at the end of the run (the summary survives -q).
_MARGINS = {"rows": 0, "cut": math.inf, "draw": math.inf, "under": 0, "ties": 0}
_IN_GPU_TEST = [False]
_TIE_TEST = [False]  # a test whose rows put a prefix exactly on its threshold on purpose
_TIGHT = 1e-12


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: takes more than a few seconds on the CPU")
    config.addinivalue_line("markers", "ties: rows built with zero cut or draw margin on purpose")


def pytest_runtest_setup(item):
    _IN_GPU_TEST[0] = item.get_closest_marker("gpu") is not None
    _TIE_TEST[0] = item.get_closest_marker("ties") is not None


def pytest_runtest_teardown(item):
    _IN_GPU_TEST[0] = False
    _TIE_TEST[0] = False


def _record(dg):
    if not _IN_GPU_TEST[0]:
        return
    if _TIE_TEST[0]:
        _MARGINS["ties"] += 1
        return
    _MARGINS["rows"] += 1
    _MARGINS["cut"] = min(_MARGINS["cut"], dg["cut_margin"])
    _MARGINS["draw"] = min(_MARGINS["draw"], dg["draw_margin"])
    if min(dg["cut_margin"], dg["draw_margin"]) < _TIGHT:
        _MARGINS["under"] += 1


def pytest_terminal_summary(terminalreporter):
    if _MARGINS["rows"] == 0:
        return
    terminalreporter.write_line(
        f"sampled-row margins: {_MARGINS['rows']} device rows checked against the oracle; smallest cut "
        f"margin {_MARGINS['cut']:.3e}, smallest draw margin {_MARGINS['draw']:.3e}; rows with a "
        f"margin under {_TIGHT:g}: {_MARGINS['under']}; rows built with a zero margin on purpose (and "
        f"checked the same way): {_MARGINS['ties']}")


@pytest.fixture(scope="session")
def oracle():
    import oracle as O
    O.lib()
    if not getattr(O.sample_token, "_records_margins", False):
        plain = O.sample_token

        def sample_token(*args, **kwargs):
            if not _IN_GPU_TEST[0]:
                return plain(*args, **kwargs)
            asked = kwargs.pop("diag", False)
            tok, dg = plain(*args, diag=True, **kwargs)
            if dg["want"] > 0:  # a sampled row (greedy rows carry no margins)
                _record(dg)
            return (tok, dg) if asked else tok

        sample_token._records_margins = True
        O.sample_token = sample_token
    return O


@pytest.fixture(scope="session")
def reference():
    import oracle as O
    if not O.Reference.available():
        pytest.skip("oracle/_ref/libref.so not built (needs the reference checkout)")
    return O.Reference()


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "sampling_golden.json")) as f:
        return json.load(f)
