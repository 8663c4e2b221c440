"""The VALU span-attention kernel (the measured alternative to the MFMA
kernel, selected with MAC_AMD_ATTN_IMPL=valu once per process) keeps parity
with the oracle.  It runs in one child process because the selection is
read once."""

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu


def test_valu_kernel_matches_oracle():
    here = os.path.dirname(os.path.abspath(__file__))
    env = dict(os.environ, MAC_AMD_ATTN_IMPL="valu")
    r = subprocess.run([sys.executable, "-u", os.path.join(here, "valu_variant_check.py")], env=env,
                       capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "VALU variant OK" in r.stdout
