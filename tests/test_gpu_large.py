"""GPU checks at the full measured sizes.

The oracle cannot evaluate a 32768-token sequence in a test's time budget, so the
long-context workload is checked on a seeded sample of query rows (O, lse and dQ
from the closed form restricted to those rows, all keys) plus size-independent
invariants that hold for every workload.

dQ of the long-context workload (one q/k channel scaled x20, near one-hot softmax
rows) is compared with the closed form evaluated on the operands a flash backward
receives and multiplies: the saved lse and bf16 O (delta = rowsum(dO * O)), and dS
rounded to bf16 before the dS K product (the reference's FA4 wrapper does the
same). Near one-hot rows amplify a 2e-4 lse difference, which fp32 accumulation
of |S| ~ 300 logits can leave, into ~0.2 of dQ on the x20 channel, so the saved
lse is the operand to compare against. On these
rows those two roundings alone move dQ by 0.44 from the all-fp32 closed form
(0.40 from O, 0.19 from dS), so the all-fp32 comparison is reported and bounded by
1.5 x that emulated shift plus 5e-2, while the operand-matched comparison keeps 5e-2.

Invariants:

* sum over the keys of a sequence of dK is zero: dK = scale * dS^T Q and every
  row of dS sums to zero (sum_j P_ij (dP_ij - delta_i) = 0);
* sum over the keys of a sequence of dV equals the sum over the sequence's
  active queries of dO, summed over the q-heads of each kv head (rows of P sum to 1).

Tolerances (max-abs): O 2e-2, dQ 5e-2, lse 1e-2; invariants relative to the
magnitude of the summed terms.
"""

import math

import pytest
import torch

from mimir_amd import prefixlm_attn_fwd
from mimir_amd.workloads import make_config
from oracle.prefixlm_oracle import prefixlm_mask

pytestmark = pytest.mark.gpu


def run(case, device):
    c = case.to(device)
    q, k, v = (t.clone().requires_grad_(True) for t in (c.q, c.k, c.v))
    out, lse = prefixlm_attn_fwd(q, k, v, c.is_causal, c.prefix_lens, c.causal_lens, c.cu_seqlens, c.total_seqlen,
                                 c.numseqs, c.max_seqlen_all)
    out.backward(c.dout)
    torch.cuda.synchronize()
    return out.detach(), lse, q.grad, k.grad, v.grad


def check_invariants(case, dk, dv, label):
    hq, hkv = case.q.shape[1], case.k.shape[1]
    G = hq // hkv
    dof = case.dout.float()
    starts = case.cu_seqlens[: len(case.seq_lens)].tolist()
    worst_k = worst_v = 0.0
    for s0, n in zip(starts, case.seq_lens):
        sk = dk[s0:s0 + n].double().sum(0).cpu()                       # [Hkv, D]
        mag_k = dk[s0:s0 + n].double().abs().sum(0).cpu().clamp_min(1.0)
        worst_k = max(worst_k, (sk.abs() / mag_k).max().item())
        sv = dv[s0:s0 + n].double().sum(0).cpu()
        ref = dof[s0:s0 + n].double().sum(0).reshape(hkv, G, -1).sum(1)
        mag_v = dv[s0:s0 + n].double().abs().sum(0).cpu().clamp_min(1.0)
        worst_v = max(worst_v, ((sv - ref).abs() / mag_v).max().item())
    print(f"[invariants] {label} dK zero-sum rel {worst_k:.2e}  dV = sum dO rel {worst_v:.2e}", flush=True)
    assert worst_k < 2e-2 and worst_v < 2e-2


@pytest.mark.parametrize("idx", [2, 3, 5])
def test_gradient_invariants(device, idx):
    case = make_config(idx, seed=0)
    _, _, _, dk, dv = run(case, device)
    check_invariants(case, dk, dv, f"cfg{idx}")


def test_long_context_sampled_rows(device):
    case = make_config(4, seed=0)
    out, lse, dq, dk, dv = run(case, device)
    check_invariants(case, dk, dv, "cfg4")

    n, p = case.seq_lens[0], case.prefixes[0]
    hq, hkv, d = case.q.shape[1], case.k.shape[1], case.q.shape[2]
    G = hq // hkv
    scale = 1.0 / math.sqrt(d)
    gen = torch.Generator().manual_seed(4)
    rows = torch.cat([torch.tensor([0, p - 1, p, n - 1]), torch.randint(0, n, (28,), generator=gen)]).unique()
    qf = case.q.float()[rows]                           # [R, Hq, D]
    kf = case.k.float().repeat_interleave(G, dim=1)     # [n, Hq, D]
    vf = case.v.float().repeat_interleave(G, dim=1)
    dof = case.dout.float()[rows]
    worst = {"o": 0.0, "lse": 0.0, "dq": 0.0}
    for h in range(hq):
        s = (qf[:, h] @ kf[:, h].T) * scale                              # [R, n]
        allowed = torch.arange(n)[None, :] < torch.clamp(rows[:, None] + 1, min=p)
        s = s.masked_fill(~allowed, float("-inf"))
        ref_lse = torch.logsumexp(s, dim=1)
        pr = torch.exp(s - ref_lse[:, None])
        o = pr @ vf[:, h]
        dp = dof[:, h] @ vf[:, h].T
        o_stored = out[rows, h].float().cpu()
        dq_fp32 = (pr * (dp - (dof[:, h] * o).sum(1, keepdim=True)) * scale) @ kf[:, h]
        pr_saved = torch.exp(s - lse[h, rows].cpu()[:, None])
        ds = pr_saved * (dp - (dof[:, h] * o_stored).sum(1, keepdim=True))
        dq_bf16o = (ds.bfloat16().float() @ kf[:, h]) * scale
        ds_ref = pr * (dp - (dof[:, h] * o.bfloat16().float()).sum(1, keepdim=True))
        dq_ref_o = (ds_ref.bfloat16().float() @ kf[:, h]) * scale
        got = dq[rows, h].float().cpu()
        worst["o"] = max(worst["o"], (o_stored - o).abs().max().item())
        worst["lse"] = max(worst["lse"], (lse[h, rows].cpu() - ref_lse).abs().max().item())
        worst["dq"] = max(worst["dq"], (got - dq_bf16o).abs().max().item())
        worst["dq_vs_fp32"] = max(worst.get("dq_vs_fp32", 0.0), (got - dq_fp32).abs().max().item())
        worst["intrinsic"] = max(worst.get("intrinsic", 0.0), (dq_ref_o - dq_fp32).abs().max().item())
    print(f"[cfg4 sampled rows] {worst} rows={rows.numel()}", flush=True)
    assert worst["o"] <= 2e-2 and worst["lse"] <= 1e-2 and worst["dq"] <= 5e-2, worst
    assert worst["dq_vs_fp32"] <= 1.5 * worst["intrinsic"] + 5e-2, worst
    # the sampled mask agrees with the reference mask statement
    assert torch.equal(prefixlm_mask(n, p, False)[rows[:4]], (torch.arange(n)[None, :] <
                                                             torch.clamp(rows[:4, None] + 1, min=p)))
