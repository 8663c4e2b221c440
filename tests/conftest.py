import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(REPO, "tests"), os.path.join(REPO, "mac-attention_amd"), REPO):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libmac_hip.so")


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """Decisions excused from exact parity (similarity within 1e-6 of the
    threshold), logged by helpers.near_threshold_heads."""
    try:
        from helpers import NEAR_THRESHOLD_BAND, NEAR_THRESHOLD_LOG, PARITY_LOG
    except Exception:  # pragma: no cover
        return
    if PARITY_LOG:
        terminalreporter.write_sep("-", "decode output vs oracle: largest relative L2 error per case")
        for what, v in sorted(PARITY_LOG.items()):
            terminalreporter.write_line(f"{v:.3e}  {what}")
    if NEAR_THRESHOLD_LOG:
        terminalreporter.write_sep("-", f"near-threshold decisions (|s - thr| <= {NEAR_THRESHOLD_BAND:g}), "
                                        "logged and excused from exact parity")
        for e in NEAR_THRESHOLD_LOG:
            terminalreporter.write_line(str(e))
