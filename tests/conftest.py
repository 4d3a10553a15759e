import os
import sys
from pathlib import Path

import pytest

# The library reads its phase-1 test knobs (MHCPRE_FORCE_PATH,
# MHCPRE_SPIN_LIMIT, MHCPRE_ROWS_B, MHCPRE_ROWS_PARTIALS) only under this gate.
os.environ["MHCPRE_TESTING"] = "1"

ROOT = Path(__file__).resolve().parents[1]
for p in (str(ROOT), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (gfx950)")


def pytest_terminal_summary(terminalreporter):
    """One line on how much of the hIn tolerance the GPU parity checks used:
    elements more than 1 ulp from the oracle's hIn (each within the bound the
    tolerated hPre difference propagates, tests/helpers.py)."""
    from helpers import HIN_STATS

    if HIN_STATS["checks"]:
        terminalreporter.write_line(
            f"hIn vs oracle: {HIN_STATS['beyond']} of {HIN_STATS['elements']} elements beyond "
            f"1 ulp (max {HIN_STATS['max_ulp']} ulp) over {HIN_STATS['checks']} checks, each "
            f"within the hPre-propagation bound")
    if HIN_STATS["attributed"]:
        terminalreporter.write_line(
            f"hIn beyond 1 ulp vs an fp64 evaluation: {HIN_STATS['attributed']} elements, device "
            f"closer {HIN_STATS['device_closer']}, oracle closer {HIN_STATS['oracle_closer']}, "
            f"tied {HIN_STATS['tied']}; sum of |hIn - fp64| / |fp64|: device "
            f"{HIN_STATS['device_hin_l1']:.4g}, oracle {HIN_STATS['oracle_hin_l1']:.4g}; "
            f"|hPre - fp64| on those rows, max: device {HIN_STATS['device_pre_err']:.3e}, "
            f"oracle {HIN_STATS['oracle_pre_err']:.3e}, mean: device "
            f"{HIN_STATS['device_pre_l1'] / max(HIN_STATS['pre_count'], 1):.3e}, oracle "
            f"{HIN_STATS['oracle_pre_l1'] / max(HIN_STATS['pre_count'], 1):.3e}")


@pytest.fixture(scope="session")
def pkg():
    from __graft_entry__ import load_package

    return load_package()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle

    return oracle


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")
