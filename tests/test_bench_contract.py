"""bench.py contract checks that need no GPU."""

import json
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_headline_pmc_summary_is_parsable():
    sys.path.insert(0, REPO)
    import bench

    args = bench.parse_args.__globals__["argparse"].Namespace(hkv=8, batch=64, ctx=130048, ring=32, hit=0.8,
                                                               front_sink=0)
    traffic, src = bench.pmc_traffic(args)
    assert src == "profiles/span_attention_config3_gqa4_hit0.8_pmc.txt"
    assert 6.9e9 < traffic < 7.2e9
