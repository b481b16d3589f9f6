"""CPU checks of bench.py's byte accounting for the score-gradient hand-off.

``dscore_blocks`` counts the 32 x 32 (query, key) blocks per head that hold an
attended pair, i.e. the dS blocks the dK / dV kernel stores and the dQ kernel
reads; it is pinned here against a brute-force count over the oracle's mask.
"""

import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402
from mimir_amd.workloads import make_case  # noqa: E402
from oracle.prefixlm_oracle import prefixlm_mask  # noqa: E402


def _brute_force_blocks(case) -> int:
    cu = case.cu_seqlens.tolist()
    total = 0
    for s in range(int(case.numseqs)):
        n = cu[s + 1] - cu[s]
        mask = prefixlm_mask(n, int(case.prefix_lens[s]), bool(case.is_causal))
        for qa in range(0, n, 32):
            for ka in range(0, n, 32):
                total += int(bool(mask[qa:qa + 32, ka:ka + 32].any()))
    return total


@pytest.mark.parametrize("seq_lens,prefixes,causal", [
    ([300], [100], False),
    ([512, 200, 1, 77], [0, 200, 1, 30], False),
    ([129, 64, 65, 1, 2], [129, 0, 33, 0, 2], False),
    ([256, 300], [17, 299], True),
    ([33, 31, 32], [32, 31, 0], False),
])
def test_dscore_blocks_match_the_mask(seq_lens, prefixes, causal):
    case = make_case(seq_lens, prefixes, 2, 1, 64, seed=0, is_causal=causal)
    assert bench.dscore_blocks(case) == _brute_force_blocks(case)
