"""GPU parity of the HIP prefix-LM kernels against the CPU oracle.

Every case runs the product path (``mimir_amd.prefixlm_attn_fwd`` -> C ABI ->
HIP kernels) on seeded inputs and compares with the oracle's restatement of the
reference masked-SDPA path evaluated in fp32 on the same (bf16-rounded) inputs.

Tolerances (max-abs, written here as the contract):
  bf16 kernels: O <= 2e-2, dQ/dK/dV <= 5e-2, lse <= 1e-2
  fp32 kernel:  O <= 1e-5, lse <= 1e-5; fp32 gradients <= 1e-4
"""

import ctypes

import pytest
import torch

from mimir_amd import prefixlm_attn_fwd
from mimir_amd.workloads import make_case, make_config
from oracle.prefixlm_oracle import dense_backward, dense_forward, dense_lse

pytestmark = pytest.mark.gpu

TOL = {
    torch.bfloat16: dict(o=2e-2, grad=5e-2, lse=1e-2),
    torch.float32: dict(o=1e-5, grad=1e-4, lse=1e-5),
}


def run_gpu(case, device, backward=True):
    c = case.to(device)
    q = c.q.clone().requires_grad_(backward)
    k = c.k.clone().requires_grad_(backward)
    v = c.v.clone().requires_grad_(backward)
    out, lse = prefixlm_attn_fwd(q, k, v, c.is_causal, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                 c.total_seqlen, c.numseqs, c.max_seqlen_all)
    res = {"o": out.detach().float().cpu(), "lse": lse.detach().float().cpu()}
    if backward:
        out.backward(c.dout)
        res.update(dq=q.grad.float().cpu(), dk=k.grad.float().cpu(), dv=v.grad.float().cpu())
    torch.cuda.synchronize()
    return res


def run_oracle(case, backward=True):
    qf, kf, vf, dof = (t.float() for t in (case.q, case.k, case.v, case.dout))
    args = case.oracle_args()
    o = dense_forward(qf, kf, vf, case.is_causal, *args)
    res = {"o": o, "lse": dense_lse(qf, kf, case.is_causal, *args)}
    if backward:
        dq, dk, dv = dense_backward(qf, kf, vf, o, dof, case.is_causal, *args)
        res.update(dq=dq, dk=dk, dv=dv)
    return res


def maxdiff(a, b):
    fin = torch.isfinite(b)
    assert torch.equal(fin, torch.isfinite(a)), "non-finite pattern differs"
    return (a[fin] - b[fin]).abs().max().item() if fin.any() else 0.0


def check(case, device, backward=True, label=""):
    tol = TOL[case.q.dtype]
    got = run_gpu(case, device, backward)
    ref = run_oracle(case, backward)
    errs = {key: maxdiff(got[key], ref[key]) for key in ref}
    print(f"[parity] {label} {case.q.dtype} T={case.T} seqs={case.seq_lens[:8]} p={case.prefixes[:8]} errs={errs}",
          flush=True)
    assert errs["o"] <= tol["o"], errs
    assert errs["lse"] <= tol["lse"], errs
    if backward:
        for key in ("dq", "dk", "dv"):
            assert errs[key] <= tol["grad"], errs
    # rows outside every sequence / at or after total_seqlen are exactly zero
    total = int(case.total_seqlen)
    if total < case.T:
        assert torch.count_nonzero(got["o"][total:]) == 0
        assert torch.isneginf(got["lse"][:, total:]).all()
        if backward:
            assert torch.count_nonzero(got["dq"][total:]) == 0
    return got


SMALL = [
    # (seq_lens, prefixes, hq, hkv, d, pad_to, is_causal)
    ([300], [100], 2, 2, 128, None, False),
    ([512, 200, 1, 77], [0, 200, 1, 30], 8, 2, 128, 1000, False),
    ([129, 64, 65, 1, 2], [129, 0, 33, 0, 2], 4, 4, 128, None, False),
    ([700], [650], 4, 1, 128, None, False),
    ([256, 300], [17, 299], 4, 2, 128, None, True),
    ([300], [100], 2, 2, 64, None, False),
    ([512, 200, 1, 77], [0, 200, 1, 30], 8, 2, 64, 1000, False),
    ([1000, 24], [500, 0], 8, 8, 64, None, False),
    ([190, 64, 3], [64, 64, 0], 16, 2, 128, 300, False),
]


@pytest.mark.parametrize("idx", range(len(SMALL)))
def test_bf16_small(device, idx):
    seq_lens, prefixes, hq, hkv, d, pad_to, causal = SMALL[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=idx, dtype=torch.bfloat16, pad_to=pad_to,
                     is_causal=causal)
    check(case, device, label=f"small{idx}")


def _random_shape(seed):
    """A seeded random packing: 1-6 documents of 1..700 tokens, prefixes anywhere in [0, n]
    (often 0 or n), GQA ratio 1/2/4/8, head_dim 64 or 128, sometimes is_causal or padding rows."""
    g = torch.Generator().manual_seed(1000 + seed)
    r = lambda lo, hi: int(torch.randint(lo, hi + 1, (1,), generator=g))
    ndoc = r(1, 6)
    seq_lens = [r(1, 700) for _ in range(ndoc)]
    prefixes = []
    for n in seq_lens:
        kind = r(0, 3)
        prefixes.append(0 if kind == 0 else n if kind == 1 else r(0, n))
    hkv = [1, 2, 4][r(0, 2)]
    hq = hkv * [1, 2, 4, 8][r(0, 3)]
    d = [64, 128][r(0, 1)]
    pad = sum(seq_lens) + r(0, 70) if r(0, 2) == 0 else None
    return seq_lens, prefixes, hq, hkv, d, pad, r(0, 4) == 0


@pytest.mark.parametrize("seed", range(16))
def test_bf16_random_shapes(device, seed):
    """Seeded random shapes (the edge cases above are hand-picked; these are not)."""
    seq_lens, prefixes, hq, hkv, d, pad_to, causal = _random_shape(seed)
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=seed, dtype=torch.bfloat16, pad_to=pad_to,
                     is_causal=causal)
    check(case, device, label=f"random{seed} hq={hq} hkv={hkv} d={d} causal={causal} pad={pad_to}")


@pytest.mark.parametrize("seed", range(16, 24))
def test_bf16_random_shapes_split(device, seed):
    """Further seeded random shapes with split mode "always": the split bodies (P and dS as two
    bf16 halves) of the forward and of both dK/dV kernels over the same kind of packings,
    against the same bars."""
    from mimir_amd import prefixlm as P

    seq_lens, prefixes, hq, hkv, d, pad_to, causal = _random_shape(seed)
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=seed, dtype=torch.bfloat16, pad_to=pad_to,
                     is_causal=causal)
    mode = P._split_mode
    try:
        P.set_split_mode("always")
        check(case, device, label=f"random-split{seed} hq={hq} hkv={hkv} d={d} causal={causal} pad={pad_to}")
    finally:
        P._split_mode = mode


@pytest.fixture
def dscore_limit():
    """Set the score-gradient workspace limit for one test; the default comes back after."""
    from mimir_amd import prefixlm as P

    saved = P._dscore_limit_bytes
    yield P.set_dscore_workspace_limit
    P.set_dscore_workspace_limit(saved)


@pytest.mark.parametrize("idx", [1, 3, 4, 8])
def test_bf16_recompute_dq(device, idx, dscore_limit):
    """The dQ kernel that recomputes S and dP (score-gradient hand-off off) meets the same bar."""
    dscore_limit(0)
    seq_lens, prefixes, hq, hkv, d, pad_to, causal = SMALL[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=idx, dtype=torch.bfloat16, pad_to=pad_to,
                     is_causal=causal)
    check(case, device, label=f"recompute small{idx}")


def test_dscore_handoff_matches_recompute(device, dscore_limit):
    """dK / dV are bitwise the same with and without the hand-off (the stores change no
    arithmetic); dQ from the stored dS agrees with the recomputed one to bf16 rounding of dS; a
    limit below the tiles' size falls back to the recompute, bit for bit."""
    case = make_case([900, 333, 64, 5], [450, 0, 64, 2], 8, 2, 128, seed=21, dtype=torch.bfloat16, pad_to=1400)
    dscore_limit(4 << 30)
    on = run_gpu(case, device)
    dscore_limit(0)
    off = run_gpu(case, device)
    dscore_limit(1)
    tiny = run_gpu(case, device)
    assert torch.equal(on["dk"], off["dk"]) and torch.equal(on["dv"], off["dv"])
    err = (on["dq"] - off["dq"]).abs().max().item()
    print(f"[parity] dscore hand-off vs recompute: dq max diff {err:.3g}", flush=True)
    assert err <= 1e-2
    for key in ("dq", "dk", "dv"):
        assert torch.equal(tiny[key], off[key])


@pytest.mark.parametrize("idx", [0, 1, 2, 4, 5, 6, 8])
def test_f32_small(device, idx):
    seq_lens, prefixes, hq, hkv, d, pad_to, causal = SMALL[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, seed=100 + idx, dtype=torch.float32, pad_to=pad_to,
                     is_causal=causal)
    check(case, device, label=f"f32small{idx}")


def test_config1_fp32_forward(device):
    case = make_config(1, seed=0)
    check(case, device, backward=False, label="cfg1")


@pytest.mark.parametrize("idx", [2, 3, 5])
def test_config_bf16_fwd_bwd(device, idx):
    case = make_config(idx, seed=0)
    check(case, device, label=f"cfg{idx}")


def test_strided_v_matches_contiguous(device):
    """v as the strided split of a fused gate/q/k/v projection (layers.py:183-184)."""
    case = make_case([384, 128], [100, 0], 8, 2, 128, seed=7, dtype=torch.bfloat16)
    c = case.to(device)
    T, hq, hkv, d = c.T, 8, 2, 128
    fused = torch.randn((T, 2 * hq + 2 * hkv, d), device=device, dtype=torch.bfloat16)
    fused[:, 2 * hq + hkv:] = c.v
    v_view = fused[:, 2 * hq + hkv:]
    assert not v_view.is_contiguous()
    o1, l1 = prefixlm_attn_fwd(c.q, c.k, v_view, False, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                               c.total_seqlen, c.numseqs, c.max_seqlen_all)
    o2, l2 = prefixlm_attn_fwd(c.q, c.k, c.v, False, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                               c.total_seqlen, c.numseqs, c.max_seqlen_all)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_deterministic(device):
    case = make_case([600, 300], [250, 10], 8, 2, 128, seed=3, dtype=torch.bfloat16)
    a = run_gpu(case, device)
    b = run_gpu(case, device)
    for key in a:
        assert torch.equal(a[key], b[key]), key


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_empty_batch_is_all_padding(device, dtype):
    """numseqs = 0: every row is padding (O = 0, lse = -inf, zero gradients), nothing else launched."""
    case = make_case([], [], 4, 2, 64, seed=5, dtype=dtype, pad_to=40)
    got = run_gpu(case, device)
    assert torch.count_nonzero(got["o"]) == 0 and torch.isneginf(got["lse"]).all()
    for key in ("dq", "dk", "dv"):
        assert torch.count_nonzero(got[key]) == 0, key


def test_backward_matches_its_stages(device):
    """mimir_prefixlm_bwd must equal, bitwise, its stages called one at a time."""
    import ctypes

    from mimir_amd import _capi
    from mimir_amd import prefixlm as P

    case = make_case([700, 300, 45], [350, 0, 45], 8, 2, 128, seed=11, dtype=torch.bfloat16)
    c = case.to(device)
    lib = _capi.load()
    stream = torch.cuda.current_stream(device).cuda_stream
    scale = 1.0 / 128 ** 0.5
    fp, out, lse, _kf = P.prepare_fwd(c.q, c.k, c.v, False, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                      c.total_seqlen, c.numseqs, c.max_seqlen_all, scale)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(fp), stream))
    grads = []
    for serial in (False, True):
        bp, dq, dk, dv, _kb = P.prepare_bwd(c.dout, c.q, c.k, c.v, out, lse, False, c.prefix_lens, c.causal_lens,
                                            c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, scale)
        if serial:
            for bits in (_capi.BWD_STAGE_DELTA, _capi.BWD_STAGE_DKDV, _capi.BWD_STAGE_DQ, _capi.BWD_STAGE_FILL):
                _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd_stages(ctypes.byref(bp), bits, stream))
        else:
            _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd(ctypes.byref(bp), stream))
        torch.cuda.synchronize()
        grads.append((dq.clone(), dk.clone(), dv.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d", [128, 64])
def test_graph_replay_matches_eager(device, d):
    """Forward + backward captured in a HIP graph: every replay, with eager calls between them,
    gives bitwise the eager result (the work lists, split counters and work queue are rebuilt or
    reset by the launches themselves; no memset nodes)."""
    import ctypes

    from mimir_amd import _capi
    from mimir_amd import prefixlm as P

    case = make_case([700, 300, 45], [350, 0, 45], 8, 2, d, seed=12, dtype=torch.bfloat16, pad_to=1100)
    c = case.to(device)
    lib = _capi.load()
    scale = 1.0 / d ** 0.5
    fp, out, lse, _kf = P.prepare_fwd(c.q, c.k, c.v, False, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                      c.total_seqlen, c.numseqs, c.max_seqlen_all, scale)
    bp, dq, dk, dv, _kb = P.prepare_bwd(c.dout, c.q, c.k, c.v, out, lse, False, c.prefix_lens, c.causal_lens,
                                        c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, scale)

    def step():
        stream = torch.cuda.current_stream(device).cuda_stream
        _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(fp), stream))
        _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd(ctypes.byref(bp), stream))

    step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (out, lse, dq, dk, dv)]
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        step()  # warm-up on the capture stream
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip((out, lse, dq, dk, dv), eager):
            assert torch.equal(got, ref)
        step()
        torch.cuda.synchronize()
        for got, ref in zip((out, lse, dq, dk, dv), eager):
            assert torch.equal(got, ref)


def _cut(case, total):
    """The same batch with total_seqlen ending before the last sequence's end."""
    case.total_seqlen = torch.tensor(int(total), dtype=torch.int64)
    return case


CUTS = [
    # seq_lens, prefixes, hq, hkv, d, total: where total_seqlen ends
    ([300, 500], [50, 100], 8, 2, 128, 300 + 250),   # inside the second sequence, past its prefix
    ([300, 500], [50, 400], 8, 2, 128, 300 + 250),   # inside the second sequence's prefix
    ([700], [64], 4, 1, 128, 333),                   # mid-tile, past the prefix
    ([300, 500], [50, 100], 8, 2, 64, 300 + 250),    # head_dim 64 kernels
]


@pytest.mark.parametrize("handoff", [True, False], ids=["handoff", "recompute"])
@pytest.mark.parametrize("idx", range(len(CUTS)))
def test_total_seqlen_inside_a_sequence(device, idx, handoff, dscore_limit):
    """total_seqlen ending inside a sequence: rows from total on are outputs of zero (O, dQ)
    and carry no gradient, while keys there remain keys of the earlier rows that see them
    (dense.py:79-80).  Keys past the last active query in the causal part get dK = dV = 0."""
    dscore_limit((4 << 30) if handoff else 0)
    seq_lens, prefixes, hq, hkv, d, total = CUTS[idx]
    case = _cut(make_case(seq_lens, prefixes, hq, hkv, d, seed=40 + idx, dtype=torch.bfloat16), total)
    check(case, device, label=f"cut{idx} total={total} handoff={handoff}")


def test_understated_max_seqlen_all(device):
    """max_seqlen_all smaller than a sequence: the validated call raises ValueError; without
    validation the result is still correct (the tile lists do not depend on it, and dQ falls
    back from the score-gradient region, which it sizes, to the recompute)."""
    from mimir_amd import prefixlm as P

    case = make_case([900, 300], [400, 0], 8, 2, 128, seed=50, dtype=torch.bfloat16)
    case.max_seqlen_all = torch.tensor(300, dtype=torch.int64)
    saved = P._validate_metadata
    try:
        P.set_validate_metadata(True)
        with pytest.raises(ValueError, match="max_seqlen_all"):
            run_gpu(case, device)
        P.set_validate_metadata(False)
        check(case, device, label="max_seqlen_all understated")
    finally:
        P._validate_metadata = saved


@pytest.fixture
def fwd_min_workspace():
    """The forward with its minimum workspace (no key-range parts), so that the only large
    float32 allocations of a step are the backward's."""
    from mimir_amd import prefixlm as P

    saved = P._key_chunks
    P.set_key_chunks(False)
    yield
    P.set_key_chunks(saved)


def test_workspace_oom_falls_back_to_recompute(device, monkeypatch, fwd_min_workspace):
    """If the backward workspace with the score-gradient region cannot be allocated, the
    backward runs with the small workspace and the recomputing dQ: same dK / dV bit for
    bit, dQ within the bar."""
    from mimir_amd import prefixlm as P

    from mimir_amd import _capi

    case = make_case([900, 333], [450, 0], 8, 2, 128, seed=51, dtype=torch.bfloat16)
    base = run_gpu(case, device)
    # the workspace without the region: anything larger is the hand-off request
    small = _capi.load().mimir_prefixlm_bwd_workspace_bytes(case.T, 8, 2, 900)
    real_empty = torch.empty
    refused = []

    def empty(*shape, **kw):
        n = 1
        for s in (shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape):
            n *= int(s)
        if kw.get("dtype") is torch.float32 and n * 4 > small and not refused:
            refused.append(n)
            raise torch.cuda.OutOfMemoryError("refused by the test")
        return real_empty(*shape, **kw)

    monkeypatch.setattr(P.torch, "empty", empty)
    got = run_gpu(case, device)
    monkeypatch.undo()
    assert refused, "the hand-off workspace was never requested"
    assert torch.equal(got["dk"], base["dk"]) and torch.equal(got["dv"], base["dv"])
    assert (got["dq"] - base["dq"]).abs().max().item() <= 1e-2
    check(case, device, label="after OOM fallback")


def test_dscore_region_bounded_by_free_memory(device, monkeypatch, fwd_min_workspace):
    """A large score-gradient region is requested only while it fits half of the free device
    memory: with the free memory reported just below twice the region the backward allocates
    the small workspace and recomputes dQ (dK / dV bit for bit, dQ within the bar); just above
    it, the workspace holds the region and dQ is the hand-off's, bit for bit."""
    from mimir_amd import prefixlm as P
    from mimir_amd import _capi

    case = make_case([900, 333], [450, 0], 8, 2, 128, seed=52, dtype=torch.bfloat16)
    lib = _capi.load()
    b = _capi.BwdParams()
    b.total_tokens, b.num_q_heads, b.num_kv_heads, b.numseqs, b.max_seqlen_all = case.T, 8, 2, 2, 900
    b.head_dim, b.dtype, b.dscore_limit_bytes = 128, _capi.DTYPE_BFLOAT16, 1 << 40
    region = int(lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(b)))
    small = int(lib.mimir_prefixlm_bwd_workspace_bytes(case.T, 8, 2, 900))
    assert region > 0
    base = run_gpu(case, device)  # hand-off (plenty of free memory)
    real_empty = torch.empty
    for free, handoff in ((2 * region - 2, False), (2 * region + 2, True)):
        requested = []

        def empty(*shape, **kw):
            if kw.get("dtype") is torch.float32:
                n = 1
                for d in (shape[0] if len(shape) == 1 and isinstance(shape[0], (tuple, list)) else shape):
                    n *= int(d)
                requested.append(n * 4)
            return real_empty(*shape, **kw)

        monkeypatch.setattr(P, "_free_device_bytes", lambda dev, f=free: f)
        monkeypatch.setattr(P, "_total_device_bytes", lambda dev: 0)  # every region counts as large
        monkeypatch.setattr(P.torch, "empty", empty)
        got = run_gpu(case, device)
        monkeypatch.undo()
        ws = max(requested)
        print(f"[free-memory bound] free {free} region {region}: workspace {ws} (small {small})", flush=True)
        assert (ws > small + region // 2) == handoff
        assert torch.equal(got["dk"], base["dk"]) and torch.equal(got["dv"], base["dv"])
        if handoff:
            assert torch.equal(got["dq"], base["dq"])
        else:
            assert (got["dq"] - base["dq"]).abs().max().item() <= 1e-2
    check(case, device, label="free-memory bound")
