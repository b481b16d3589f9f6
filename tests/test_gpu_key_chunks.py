"""GPU checks of the key-range parts of the forward and dQ kernels on small grids.

When fewer than 512 (query tile, q head) workgroups make up the forward's grid
(few heads over a short packed row, e.g. the 2-head 24k-token workload), the
work list cuts the key ranges of its heaviest query tiles into parts; each part
runs as its own workgroup and writes its unnormalized O with its running max
and sum, and the last part of a tile to arrive merges all parts in part order
and writes O and lse.  The merged result differs from the uncut forward only by
fp32 summation order, so:

* against the oracle the usual bf16 bar holds (O <= 2e-2, lse <= 1e-2);
* against the uncut forward: O within one bf16 rounding step (<= 1e-2 here,
  |O| < 1), lse <= 1e-4, the RoPE-rotated q bitwise (the parts do not touch it);
* two chunked runs agree bitwise (the merge order is fixed);
* the work list really holds cut tiles (entries with parts > 1), so each case
  exercises the merge.

The dQ kernels (from the stored score gradients, and recomputing) cut the same
way and sum their parts in part order: with one forward's O and lse, the
backward with and without dQ parts gives dK / dV bitwise and dQ within one bf16
rounding step, and the cut backward matches the oracle at the bf16 bar.
"""

import ctypes
import math

import pytest
import torch

from mimir_amd import _capi, prefixlm_attn_fwd
from mimir_amd import prefixlm as P
from mimir_amd.workloads import make_case, make_config
from oracle.prefixlm_oracle import chunked_forward_backward, dense_backward, dense_forward, dense_lse

pytestmark = pytest.mark.gpu

CASES = [
    # (seq_lens, prefixes, hq, hkv, d, is_causal)
    ([4000, 1500, 300], [3000, 0, 150], 2, 2, 128, False),
    ([3000, 700], [100, 700], 2, 1, 64, False),
    ([2500, 900, 1], [0, 400, 1], 4, 2, 128, True),
    ([6000], [0], 8, 8, 128, False),
    ([2000] + [17] * 300, [1200] + [5] * 300, 1, 1, 64, False),  # > 256 sequences: the walks reload them
]


@pytest.fixture
def key_chunks():
    saved = P._key_chunks
    yield
    P._key_chunks = saved


def check_plan(case, lst, hq, chunked, span_pct):
    """The query-tile list pinned against its definition: every 128-row tile of every sequence
    appears exactly once, whole (part 0 of 1, no chunk slot) or as parts 0 .. parts - 1 with
    consecutive chunk slots no other tile uses; a tile is cut exactly when the grid is small
    (tiles x Hq < 512) and its cost exceeds span = ceil(max(total cost x Hq / 512 x span_pct / 100,
    4)) (span_pct 125 for the forward's list, 100 for dQ's; cost: the
    key tiles of 64 its rows attend), into ceil(cost / span) parts (at most 16) whose key ranges the
    kernels take as: the last parts span tiles each, part 0 the rest; entries run heaviest first
    by the cost of what each runs; padding (-1) only after the last."""
    total = int(case.total_seqlen)
    cu = [int(x) for x in case.cu_seqlens[: len(case.seq_lens) + 1]]
    expect = {}
    for s, (n, p) in enumerate(zip(case.seq_lens, case.prefixes)):
        nq = max(0, min(n, total - cu[s]))
        p = 0 if case.is_causal else min(p, n)
        for t in range(-(-nq // 128)):
            expect[(s, t)] = -(-max(p, min(128 * t + 128, nq)) // 64)
    cost_total = sum(expect.values())
    small = chunked and len(expect) * hq < 512
    target = cost_total * hq / 512 * span_pct / 100.0
    span = (math.ceil(target) if target > 4.0 else 4) if small else 0
    seen, costs, slots, padding = {}, [], set(), False
    for x, y, z, w in lst.tolist():
        if x < 0:
            padding = True
            continue
        assert not padding, "an entry after the padding"
        part, parts, zspan = z & 0xFF, (z >> 8) & 0xFF, z >> 16
        c = expect[(x, y)]
        want = 1 if not small or c <= span else min(math.ceil(c / span), 16)
        assert parts == want, ((x, y), c, parts, want)
        if parts == 1:
            assert part == 0 and w == -1 and zspan == 0
            runs = c
        else:
            assert 0 <= part < parts and w >= 0 and w not in slots and zspan == span
            slots.add(w)
            # the kernels' key range of this part: [kt0, kt1) of the tile's c key tiles
            kt0 = 0 if part == 0 else c - (parts - part) * span
            kt1 = c - (parts - 1 - part) * span
            assert 0 <= kt0 < kt1 <= c
            runs = kt1 - kt0
        seen.setdefault((x, y), []).append((part, w, runs))
        costs.append(min(runs, 4095))
    assert set(seen) == set(expect)
    for key, ps in seen.items():
        ps.sort()
        assert [q for q, _, _ in ps] == list(range(len(ps)))
        assert len({w - q for q, w, _ in ps}) == 1  # consecutive slots
        assert sum(r for _, _, r in ps) == expect[key]  # the parts cover the key range once
    assert all(a >= b for a, b in zip(costs, costs[1:])), "not heaviest first"


def forward(c, chunks, case=None, **kw):
    """One forward launch through the C ABI; returns (outputs dict, cut tiles in the work list).
    With `case`, the work list is checked against its definition (check_plan)."""
    P._key_chunks = chunks
    lib = _capi.load()
    d = c.q.shape[2]
    p, out, lse, keep = P.prepare_fwd(c.q, c.k, c.v, c.is_causal, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                      c.total_seqlen, c.numseqs, c.max_seqlen_all, d ** -0.5, **kw)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    ws = keep[6]
    entries = -(-c.T // 128) + int(c.numseqs)
    if p.workspace_bytes > lib.mimir_prefixlm_fwd_workspace_bytes(c.T, int(c.numseqs), int(c.max_seqlen_all)):
        entries += 1024 // c.q.shape[1]  # the chunk slots' list entries
    lst = ws.view(torch.int32)[: 4 * entries].view(-1, 4).cpu()
    cut = int(((lst[:, 0] >= 0) & (((lst[:, 2] >> 8) & 0xFF) > 1)).sum())
    if case is not None:
        check_plan(case, lst, c.q.shape[1], chunks, 125)
    res = {"o": out.clone(), "lse": lse.clone()}
    for name, t in kw.items():
        if isinstance(t, torch.Tensor) and t.dtype == c.q.dtype:
            res[name] = t.clone()
    return res, cut


def close(a, b):
    fin = torch.isfinite(b)
    assert torch.equal(fin, torch.isfinite(a))
    return (a[fin].double() - b[fin].double()).abs().max().item() if fin.any() else 0.0


@pytest.mark.parametrize("idx", range(len(CASES)))
def test_chunked_forward(device, idx, key_chunks):
    seq_lens, prefixes, hq, hkv, d, causal = CASES[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=40 + idx, dtype=torch.bfloat16, is_causal=causal)
    c = case.to(device)
    got, cut = forward(c, True, case)
    again, _ = forward(c, True)
    plain, none = forward(c, False, case)
    print(f"[chunks] case {idx}: {cut} cut list entries; uncut run {none}", flush=True)
    assert cut > 0 and none == 0
    for key in got:
        assert torch.equal(got[key], again[key]), key
    assert close(got["o"], plain["o"]) <= 1e-2
    assert close(got["lse"], plain["lse"]) <= 1e-4
    qf, kf, vf = (t.float() for t in (case.q, case.k, case.v))
    args = case.oracle_args()
    o_ref = dense_forward(qf, kf, vf, case.is_causal, *args)
    lse_ref = dense_lse(qf, kf, case.is_causal, *args)
    errs = (close(got["o"].float().cpu(), o_ref), close(got["lse"].float().cpu(), lse_ref))
    print(f"[chunks] case {idx}: O {errs[0]:.3g} lse {errs[1]:.3g} against the oracle", flush=True)
    assert errs[0] <= 2e-2 and errs[1] <= 1e-2


def test_padded_small_grid_is_cut(device, key_chunks):
    """A padded batch: 3700 real tokens in a 40000-row tensor.  By the tensor's length alone
    (ceil(40000 / 128) x 2 heads = 626 >= 512 workgroups) the grid could not be small, but its
    query tiles (29 x 2) are few: the chunk room is sized from min(T, total_seqlen), so the
    list cuts them; the cut forward matches the oracle and leaves the padding rows zero."""
    case = make_case([3000, 700], [100, 700], 2, 1, 128, seed=49, dtype=torch.bfloat16, pad_to=40000)
    c = case.to(device)
    assert -(-c.T // 128) * 2 >= 512 and -(-int(c.total_seqlen) // 128) * 2 < 512
    got, cut = forward(c, True, case)
    print(f"[chunks] padded small grid: {cut} cut list entries", flush=True)
    assert cut > 0
    total = int(c.total_seqlen)
    assert torch.equal(got["o"][total:], torch.zeros_like(got["o"][total:]))
    assert torch.isneginf(got["lse"][:, total:]).all()
    qf, kf, vf = (t.float() for t in (case.q, case.k, case.v))
    args = case.oracle_args()
    o_ref = dense_forward(qf, kf, vf, case.is_causal, *args)
    lse_ref = dense_lse(qf, kf, case.is_causal, *args)
    errs = (close(got["o"].float().cpu(), o_ref), close(got["lse"].float().cpu(), lse_ref))
    print(f"[chunks] padded small grid: O {errs[0]:.3g} lse {errs[1]:.3g} against the oracle", flush=True)
    assert errs[0] <= 2e-2 and errs[1] <= 1e-2


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("split", [_capi.SPLIT_ALWAYS, _capi.SPLIT_NEVER], ids=["split", "plain"])
def test_chunked_forward_gate_rope(device, split, d, key_chunks):
    """Gated output, RoPE of q in the kernel (with the rotated q written out) and the P hi + lo
    split all ride on the merged accumulator: chunked and uncut agree as above (both head dims,
    so that the gated split bodies of both run)."""
    case = make_case([3500, 800], [2000, 0], 2, 2, d, seed=47, dtype=torch.bfloat16)
    c = case.to(device)
    T, hq, d = c.q.shape
    g = torch.Generator().manual_seed(48)
    pos = torch.arange(T, dtype=torch.float64)[:, None]
    freq = 10000.0 ** (-torch.arange(0, d // 2, dtype=torch.float64) / (d // 2))
    ang = torch.cat([pos * freq, pos * freq], dim=1)
    rope = (ang.cos().float().to(device), ang.sin().float().to(device))
    gate = torch.randn(T, hq, d, generator=g).to(device=device, dtype=torch.bfloat16)
    runs = []
    for chunks in (True, False):
        kw = dict(gate=gate, gated_out=torch.empty_like(c.q), out_lo=torch.empty_like(c.q), split_mode=split,
                  rope=rope, q_rope=torch.empty_like(c.q))
        runs.append(forward(c, chunks, **kw))
    (got, cut), (plain, _) = runs
    assert cut > 0
    assert torch.equal(got["q_rope"], plain["q_rope"])
    assert close(got["o"], plain["o"]) <= 1e-2
    assert close(got["gated_out"], plain["gated_out"]) <= 1e-2
    assert close(got["lse"], plain["lse"]) <= 1e-4
    if split == _capi.SPLIT_ALWAYS:  # O's low half: O - round(O), one rounding step of O at most
        assert close(got["out_lo"].float() + got["o"].float(), plain["out_lo"].float() + plain["o"].float()) <= 1e-4


def test_small_grid_workload_full_fp64(device, key_chunks):
    """The 2-head 24576-token workload (11 documents) with the key ranges of the forward and
    dQ cut: O, lse, dQ, dK and dV in full against the oracle's closed form in float64
    (evaluated on the GPU), and the gradients against those of the uncut kernels."""
    case = make_config(6, seed=0)
    c = case.to(device)
    d = c.q.shape[2]
    res = {}
    for chunks in (True, False):
        P._key_chunks = chunks
        q, k, v = (t.clone().requires_grad_(True) for t in (c.q, c.k, c.v))
        out, lse = prefixlm_attn_fwd(q, k, v, c.is_causal, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                       c.total_seqlen, c.numseqs, c.max_seqlen_all)
        out.backward(c.dout)
        torch.cuda.synchronize()
        res[chunks] = (out.detach(), lse, q.grad, k.grad, v.grad)
    _, cut = forward(c, True, case)
    assert cut > 0
    c64 = [t.to(device=device, dtype=torch.float64) for t in (case.q, case.k, case.v, case.dout)]
    o_r, lse_r, dq_r, dk_r, dv_r = chunked_forward_backward(*c64, case.is_causal, *case.oracle_args(), chunk=2048)
    e_o, e_l = close(res[True][0], o_r), close(res[True][1], lse_r)
    e_g = [close(res[True][i], r) for i, r in ((2, dq_r), (3, dk_r), (4, dv_r))]
    print(f"[chunks] 24576 x 2 heads: O {e_o:.3g} lse {e_l:.3g} dq/dk/dv {e_g} against fp64", flush=True)
    assert e_o <= 2e-2 and e_l <= 1e-2 and max(e_g) <= 5e-2
    for i, name in ((2, "dq"), (3, "dk"), (4, "dv")):
        e = close(res[True][i], res[False][i])
        print(f"[chunks] 24576 x 2 heads: {name} chunked vs uncut {e:.3g}", flush=True)
        assert e <= 5e-2, name
    assert d == 128


def _align(x):
    return (x + 255) // 256 * 256


def backward(c, out, lse, chunks, d, case=None):
    """One backward launch through the C ABI with the given forward outputs; returns
    (dq, dk, dv, cut dQ list entries); with `case` the dQ list is checked (check_plan)."""
    P._key_chunks = chunks
    lib = _capi.load()
    p, dq, dk, dv, keep = P.prepare_bwd(c.dout, c.q, c.k, c.v, out, lse, c.is_causal, c.prefix_lens, c.causal_lens,
                                        c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, d ** -0.5)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd(ctypes.byref(p), torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    cut = 0
    if p.dq_key_chunks:
        saved = p.dq_key_chunks
        p.dq_key_chunks = 0
        base = int(lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p)))
        p.dq_key_chunks = saved
        if p.workspace_bytes > base:  # the dQ list with its parts sits after the rest
            entries = -(-c.T // 128) + int(c.numseqs) + 1024 // c.q.shape[1]
            ws = keep[9].view(torch.uint8)[_align(base): _align(base) + 16 * entries].view(torch.int32)
            lst = ws.view(-1, 4).cpu()
            cut = int(((lst[:, 0] >= 0) & (((lst[:, 2] >> 8) & 0xFF) > 1)).sum())
            if case is not None:
                check_plan(case, lst, c.q.shape[1], True, 100)
    return dq.clone(), dk.clone(), dv.clone(), cut


@pytest.fixture
def dscore_limit():
    saved = P._dscore_limit_bytes
    yield
    P._dscore_limit_bytes = saved


@pytest.mark.parametrize("handoff", [True, False], ids=["handoff", "recompute"])
@pytest.mark.parametrize("idx", range(len(CASES)))
def test_chunked_dq(device, idx, handoff, key_chunks, dscore_limit):
    seq_lens, prefixes, hq, hkv, d, causal = CASES[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=50 + idx, dtype=torch.bfloat16, is_causal=causal)
    c = case.to(device)
    P.set_dscore_workspace_limit((4 << 30) if handoff else 0)
    fwd, _ = forward(c, True)
    got = backward(c, fwd["o"], fwd["lse"], True, d, case)
    again = backward(c, fwd["o"], fwd["lse"], True, d)
    plain = backward(c, fwd["o"], fwd["lse"], False, d)
    print(f"[chunks] dQ case {idx} ({'hand-off' if handoff else 'recompute'}): {got[3]} cut list entries", flush=True)
    assert got[3] > 0 and plain[3] == 0
    for a, b in zip(got[:3], again[:3]):
        assert torch.equal(a, b)
    assert torch.equal(got[1], plain[1]) and torch.equal(got[2], plain[2])
    e = close(got[0], plain[0])
    print(f"[chunks] dQ case {idx}: chunked vs uncut {e:.3g}", flush=True)
    assert e <= 1e-2
    qf, kf, vf, dof = (t.float() for t in (case.q, case.k, case.v, case.dout))
    args = case.oracle_args()
    o_ref = dense_forward(qf, kf, vf, case.is_causal, *args)
    refs = dense_backward(qf, kf, vf, o_ref, dof, case.is_causal, *args)
    errs = [close(g.float().cpu(), r) for g, r in zip(got[:3], refs)]
    print(f"[chunks] dQ case {idx}: dq/dk/dv {errs} against the oracle", flush=True)
    assert max(errs) <= 5e-2
