"""The kernel-selection switches give the same bits as the oracle.

Q4HIP_GEMM=valu keeps multi-token projections off the matrix cores (k_gemm_rows, k_gemm_q4, with
the unfused SwiGLU and RoPE launches), Q4HIP_ATTN_ROWS=0 runs a head_dim-64 prompt's attention in
three launches (scores, softmax, P.V tiles) instead of k_attn_rows, and Q4HIP_PV_TILES=0 on
k_attn_pv_list.  The library reads the switches once per process, so each case runs
tests/fallback_check.py in a child process with the switch set; that script compares prompts of
12, 40 and 150 tokens (head_dim 64 and 128), decode steps after them and a ragged batch of 12
sequences with the oracle, tokens and logits bit for bit.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("env", [{"Q4HIP_GEMM": "valu"}, {"Q4HIP_ATTN_ROWS": "0"}, {"Q4HIP_PV_TILES": "0"},
                                 {"Q4HIP_GEMM": "valu", "Q4HIP_PV_TILES": "0"}],
                         ids=["gemm-valu", "attn-three-launch", "pv-list", "both"])
def test_switch_matches_oracle(env):
    print(f"fallback switches {env}", flush=True)
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "fallback_check.py")], env=dict(os.environ, **env),
                       capture_output=True, text=True, timeout=110)
    print(r.stdout[-3000:], r.stderr[-3000:], flush=True)
    assert r.returncode == 0 and "all ok" in r.stdout, r.stdout[-1000:] + r.stderr[-1000:]
