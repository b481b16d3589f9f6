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


def _dscore_region(lib, case, limit: int) -> int:
    """The library's hand-off region for the case's sizes (0: dQ recomputes)."""
    import ctypes

    from mimir_amd import _capi

    p = _capi.BwdParams()
    T, hq, d = case.q.shape
    p.total_tokens, p.num_q_heads, p.num_kv_heads = T, hq, case.k.shape[1]
    p.numseqs, p.max_seqlen_all = int(case.numseqs), int(case.max_seqlen_all)
    p.head_dim = d
    p.dtype = _capi.DTYPE_BFLOAT16 if case.q.element_size() == 2 else _capi.DTYPE_FLOAT32
    p.dscore_limit_bytes = limit
    return int(lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)))


def test_traffic_profile_holds_the_working_kernels():
    """profiles/hbm_traffic.json (what bench.py reports as roofline.traffic) holds, for every
    profiled workload, an entry for each kernel that does a stage's work -- the names bench.py
    looks up -- and each entry is at least the bytes that kernel must move: its outputs
    plus one read of the operands it cannot skip.  (An entry of a kernel that exited at once
    holds a few KB and fails this.)"""
    import json
    import math

    from mimir_amd import _capi
    from mimir_amd import prefixlm as P
    from mimir_amd.workloads import CONFIG_NAMES, make_config

    data = json.loads((Path(__file__).resolve().parents[1] / "profiles" / "hbm_traffic.json").read_text())
    lib = _capi.load()
    recompute_tag = " (dQ recomputes: no dS hand-off)"
    by_name = {v: k for k, v in CONFIG_NAMES.items()}
    seen = set()
    for name, entries in data["workloads"].items():
        base = name[: -len(recompute_tag)] if name.endswith(recompute_tag) else name
        idx = by_name[base]
        seen.add(idx)
        case = make_config(idx, seed=0)
        T, hq, d = case.q.shape
        hkv, elem = case.k.shape[1], case.q.element_size()
        scale = 1.0 / math.sqrt(d)
        limit = 0 if name.endswith(recompute_tag) else P._dscore_limit_bytes
        handoff = _dscore_region(lib, case, limit) > 0 and not bench.auto_split(case, scale)
        names = bench.working_kernels(d, elem, handoff)
        q_bytes, kv_bytes = T * hq * d * elem, T * hkv * d * elem
        floor = {"fwd": 2 * q_bytes + 2 * kv_bytes,  # Q, K, V read, O written
                 "dkdv": 2 * q_bytes + 4 * kv_bytes,  # Q, dO, K, V read, dK, dV written
                 "dq": q_bytes + kv_bytes}  # K read, dQ written
        for stage, kernel in names.items():
            assert kernel in entries, f"{name}: no entry for {kernel}"
            assert entries[kernel]["bytes"] >= floor[stage], f"{name}: {kernel} {entries[kernel]['bytes']} B"
    assert seen == {2, 3, 4, 5, 6}
