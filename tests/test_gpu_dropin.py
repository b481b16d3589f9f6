"""The drop-in called the way Mimir2's Attention.forward calls it, on the GPU.

src/mimir/model/layers.py:183-189,223-232: q, k and v are the head splits of the
fused gqkv projection (v a strided view: token stride (2Hq + 2Hkv) * D), passed
positionally with is_causal; the three fa4_* knobs and every metadata tensor go
by keyword (``**seq_info``).  seq_info is what the training loop builds per batch:
compute_aux_seq_tensors_scalars (flash_attention_prefixlm_v2.py:21-35) as int32
device tensors plus 0-d int64 CPU scalars (src/mimir/training/loop.py:217), and for
the rocm backend the nine routing tensors of prepare_prefixlm_batch
(src/mimir/model/common.py:36-70).  The backward runs through autograd into the
gqkv gradient.

Both eager and torch.compile(fullgraph=True) -- fullgraph makes any graph break an
error, and the reference needs @torch.compiler.disable
(flash_attention_prefixlm_dispatch.py:79) exactly because its backends break the
graph.  Results are compared with the oracle (fp32 on the same bf16 inputs):
O <= 2e-2, gradients <= 5e-2 max-abs.
"""

import numpy as np
import pytest
import torch

from mimir_amd import flash_attn_varlen_prefixlm
from mimir_amd.metadata import compute_aux_seq_tensors_scalars, prefixlm_prepared_from_tensors
from mimir_amd.workloads import make_config
from oracle.prefixlm_oracle import dense_backward, dense_forward

pytestmark = pytest.mark.gpu


def seq_info_for(case, device):
    """The batch keywords of one packed row, built like the reference's data path."""
    pl = np.asarray(case.prefixes, dtype=np.int32)
    cl = np.asarray([n - p for n, p in zip(case.seq_lens, case.prefixes)], dtype=np.int32)
    tensors, scalars = compute_aux_seq_tensors_scalars(pl, cl, case.T)
    info = {k: torch.from_numpy(v.astype(np.int32)).to(device) for k, v in tensors.items()}
    info.update({k: torch.tensor(v, dtype=torch.int64) for k, v in scalars.items()})
    info.update(prefixlm_prepared_from_tensors(**info))
    return info


def attention_core(gqkv, hq, hkv, d, is_causal, **seq_info):
    """layers.py:183-189 (split of the fused projection) and 223-232 (the call)."""
    g = gqkv.view(gqkv.shape[0], 2 * hq + 2 * hkv, d)
    _gate, query, key, value = g.split((hq, hq, hkv, hkv), dim=-2)
    return flash_attn_varlen_prefixlm(query, key, value, is_causal, fa4_impl="seqused", fa4_grad_mask_impl="triton",
                                      fa4_output_combine_impl="triton", **seq_info)


def run(case, device, fn):
    T, hq, d = case.q.shape
    hkv = case.k.shape[1]
    gqkv = torch.cat([torch.zeros_like(case.q), case.q, case.k, case.v], dim=1).reshape(T, -1).to(device)
    gqkv.requires_grad_(True)
    info = seq_info_for(case, device)
    out = fn(gqkv, hq, hkv, d, case.is_causal, **info)
    out.backward(case.dout.to(device))
    torch.cuda.synchronize()
    grad = gqkv.grad.view(T, 2 * hq + 2 * hkv, d)
    return {"o": out.detach().float().cpu(), "dq": grad[:, hq:2 * hq].float().cpu(),
            "dk": grad[:, 2 * hq:2 * hq + hkv].float().cpu(), "dv": grad[:, 2 * hq + hkv:].float().cpu(),
            "dgate": grad[:, :hq].float().cpu()}


def reference(case):
    qf, kf, vf, dof = (t.float() for t in (case.q, case.k, case.v, case.dout))
    o = dense_forward(qf, kf, vf, case.is_causal, *case.oracle_args())
    dq, dk, dv = dense_backward(qf, kf, vf, o, dof, case.is_causal, *case.oracle_args())
    return {"o": o, "dq": dq, "dk": dk, "dv": dv}


def check(got, ref, label):
    errs = {k: (got[k] - ref[k]).abs().max().item() for k in ref}
    print(f"[dropin] {label} errs={errs}", flush=True)
    assert errs["o"] <= 2e-2, errs
    assert max(errs["dq"], errs["dk"], errs["dv"]) <= 5e-2, errs
    assert torch.count_nonzero(got["dgate"]) == 0  # the gate does not enter the attention call


@pytest.mark.parametrize("idx", [2, 3])
def test_dropin_eager_matches_oracle(device, idx):
    case = make_config(idx, seed=0)
    check(run(case, device, attention_core), reference(case), f"eager cfg{idx}")


@pytest.mark.timeout(600)
@pytest.mark.parametrize("idx", [2, 3])
def test_dropin_compiled_fullgraph_matches_eager(device, idx):
    """torch.compile(fullgraph=True) over the split + call + autograd: traced through the custom
    ops' fake kernels with no graph break, and numerically the eager result (the same kernels run)."""
    import torch._dynamo

    torch._dynamo.reset()
    case = make_config(idx, seed=0)
    compiled = torch.compile(attention_core, fullgraph=True, dynamic=False)
    got = run(case, device, compiled)
    check(got, reference(case), f"compiled cfg{idx}")
    eager = run(case, device, attention_core)
    for key in ("o", "dq", "dk", "dv"):
        assert torch.equal(got[key], eager[key]), key


def test_routing_tensors_match_their_definition(device):
    """The routing keywords passed above are the reference's (flash_attention_prefixlm_common.py:87-133):
    checked element by element against the per-token definition on a ragged batch."""
    case = make_config(3, seed=0)
    info = seq_info_for(case, device)
    pos, pref, act = [], [], []
    for n, p in zip(case.seq_lens, case.prefixes):
        pos += list(range(n))
        pref += [i < p for i in range(n)]
        act += [n - p > 0] * n
    pref, act = torch.tensor(pref), torch.tensor(act)
    idx = torch.arange(len(pos))
    assert torch.equal(info["prefix_mask"].cpu(), pref)
    assert torch.equal(info["causal_mask"].cpu(), ~pref & act)
    assert torch.equal(info["prefix_idx"].cpu(), idx[pref])
    assert torch.equal(info["causal_idx"].cpu(), idx[~pref & act])
    assert torch.equal(info["active_key_idx"].cpu(), idx[act])
    assert info["prefix_cu_seqlens"].cpu().tolist() == [0] + np.cumsum(case.prefixes).tolist()
