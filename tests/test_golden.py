"""Golden fixtures (fp64 brute force, tests/golden/make_golden.py): the oracle
reproduces them on the CPU, and the HIP kernels reproduce them on the GPU."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.prefixlm_oracle import dense_backward, dense_forward, dense_lse

GOLDEN = sorted((Path(__file__).parent / "golden").glob("*.npz"))


def load(path):
    z = np.load(path)  # allow_pickle=False (default): data only
    t = {k: torch.from_numpy(z[k]) for k in ("q", "k", "v", "dout", "prefix_lens", "causal_lens", "cu_seqlens")}
    meta = dict(total_seqlen=torch.tensor(int(z["total_seqlen"])), numseqs=torch.tensor(int(z["numseqs"])),
                max_seqlen_all=torch.tensor(int(z["max_seqlen_all"])), is_causal=bool(z["is_causal"]))
    ref = {k: torch.from_numpy(z[k]) for k in ("o", "lse", "dq", "dk", "dv")}
    return t, meta, ref


def test_fixtures_present():
    assert len(GOLDEN) >= 3


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_oracle_reproduces_golden(path):
    t, m, ref = load(path)
    q, k, v, do = (t[x].double() for x in ("q", "k", "v", "dout"))
    args = (t["prefix_lens"], t["causal_lens"], t["cu_seqlens"], m["total_seqlen"], m["numseqs"])
    o = dense_forward(q, k, v, m["is_causal"], *args)
    torch.testing.assert_close(o, ref["o"], atol=1e-12, rtol=0)
    lse = dense_lse(q, k, m["is_causal"], *args)
    torch.testing.assert_close(lse, ref["lse"], atol=1e-12, rtol=0)
    dq, dk, dv = dense_backward(q, k, v, o, do, m["is_causal"], *args)
    for name, got in (("dq", dq), ("dk", dk), ("dv", dv)):
        torch.testing.assert_close(got, ref[name], atol=1e-11, rtol=0)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_kernels_reproduce_golden(device, path, dtype):
    from mimir_amd import prefixlm_attn_fwd

    # bf16: O 2e-2, grads 5e-2, lse 1e-2; fp32: O / lse 1e-5, grads 1e-4 (max-abs)
    tol = dict(o=2e-2, lse=1e-2, g=5e-2) if dtype == torch.bfloat16 else dict(o=1e-5, lse=1e-5, g=1e-4)
    t, m, ref = load(path)
    q, k, v = (t[x].to(device=device, dtype=dtype).requires_grad_(True) for x in ("q", "k", "v"))
    meta = [t["prefix_lens"].to(device), t["causal_lens"].to(device), t["cu_seqlens"].to(device)]
    out, lse = prefixlm_attn_fwd(q, k, v, m["is_causal"], *meta, m["total_seqlen"], m["numseqs"], m["max_seqlen_all"])
    out.backward(t["dout"].to(device=device, dtype=dtype))
    torch.cuda.synchronize()
    fin = torch.isfinite(ref["lse"])
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    err = {
        "o": (out.detach().double().cpu() - ref["o"]).abs().max().item(),
        "lse": (lse.double().cpu()[fin] - ref["lse"][fin]).abs().max().item(),
        "dq": (q.grad.double().cpu() - ref["dq"]).abs().max().item(),
        "dk": (k.grad.double().cpu() - ref["dk"]).abs().max().item(),
        "dv": (v.grad.double().cpu() - ref["dv"]).abs().max().item(),
    }
    print(f"[golden] {path.stem} {dtype} {err}", flush=True)
    assert err["o"] <= tol["o"] and err["lse"] <= tol["lse"], err
    assert max(err["dq"], err["dk"], err["dv"]) <= tol["g"], err
