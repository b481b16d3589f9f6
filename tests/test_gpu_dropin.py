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


def seq_info_for(case, device, mark_dynamic=False):
    """The batch keywords of one packed row, built like the reference's data path; with
    ``mark_dynamic`` the routing tensors are marked dynamic as prepare_prefixlm_batch does
    (src/mimir/model/common.py:64-69), so a compiled step is not specialized on a packing."""
    pl = np.asarray(case.prefixes, dtype=np.int32)
    cl = np.asarray([n - p for n, p in zip(case.seq_lens, case.prefixes)], dtype=np.int32)
    tensors, scalars = compute_aux_seq_tensors_scalars(pl, cl, case.T)
    info = {k: torch.from_numpy(v.astype(np.int32)).to(device) for k, v in tensors.items()}
    info.update({k: torch.tensor(v, dtype=torch.int64) for k, v in scalars.items()})
    routing = prefixlm_prepared_from_tensors(**info)
    if mark_dynamic:
        for t in routing.values():
            torch._dynamo.mark_dynamic(t, 0)
    info.update(routing)
    return info


def attention_core(gqkv, hq, hkv, d, is_causal, **seq_info):
    """layers.py:183-189 (split of the fused projection) and 223-232 (the call)."""
    g = gqkv.view(gqkv.shape[0], 2 * hq + 2 * hkv, d)
    _gate, query, key, value = g.split((hq, hq, hkv, hkv), dim=-2)
    return flash_attn_varlen_prefixlm(query, key, value, is_causal, fa4_impl="seqused", fa4_grad_mask_impl="triton",
                                      fa4_output_combine_impl="triton", **seq_info)


def run(case, device, fn, mark_dynamic=False):
    T, hq, d = case.q.shape
    hkv = case.k.shape[1]
    gqkv = torch.cat([torch.zeros_like(case.q), case.q, case.k, case.v], dim=1).reshape(T, -1).to(device)
    gqkv.requires_grad_(True)
    info = seq_info_for(case, device, mark_dynamic)
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


@pytest.mark.timeout(900)
def test_dropin_compiled_once_across_packings(device):
    """Mimir2's training step is compiled once with dynamic=False (src/mimir/training/steps.py:299)
    and fed a new packing every batch, its routing tensors marked dynamic
    (src/mimir/model/common.py:64-69).  Two packings of the same 16384 tokens (different document
    lengths, counts and prefixes) run through one compiled function: Dynamo compiles a single frame
    (no recompilation for the second packing), and each packing matches the oracle."""
    import torch._dynamo
    from torch._dynamo.testing import CompileCounterWithBackend

    torch._dynamo.reset()
    counter = CompileCounterWithBackend("inductor")
    compiled = torch.compile(attention_core, backend=counter, fullgraph=True, dynamic=False)
    cases = [make_config(3, seed=s) for s in (0, 1)]
    assert cases[0].T == cases[1].T and cases[0].seq_lens != cases[1].seq_lens
    for s, case in enumerate(cases):
        check(run(case, device, compiled, mark_dynamic=True), reference(case), f"compiled packing {s}")
        print(f"[dropin] packing {s}: {len(case.seq_lens)} documents, Dynamo frames compiled so far "
              f"{counter.frame_count}", flush=True)
    assert counter.frame_count == 1


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


def test_low_output_half_memory(device):
    """With split mode "auto" (the default) every bf16 call keeps an O-sized low half of its
    output for the backward; "never" keeps none.  A stack of four chained calls held for the
    backward (each output is the next call's query) shows the cost: exactly 4 x T x Hq x D x 2
    bytes more held with "auto", and the same outputs on this plain input (auto does not split)."""
    from mimir_amd import prefixlm as P

    case = make_config(2, seed=0)
    c = case.to(device)
    T, hq, d = c.q.shape
    layers = 4
    held, peak, outs = {}, {}, {}
    mode = P._split_mode
    try:
        for m in ("auto", "never"):
            P.set_split_mode(m)
            q = c.q.clone().requires_grad_(True)
            torch.cuda.synchronize()
            base = torch.cuda.memory_allocated()
            torch.cuda.reset_peak_memory_stats()
            h = q
            for _ in range(layers):
                h = flash_attn_varlen_prefixlm(h, c.k, c.v, False, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                               c.total_seqlen, c.numseqs, c.max_seqlen_prefix, c.max_seqlen_causal,
                                               c.max_seqlen_all)
            torch.cuda.synchronize()
            held[m] = torch.cuda.memory_allocated() - base
            peak[m] = torch.cuda.max_memory_allocated() - base
            h.backward(c.dout)
            outs[m] = (h.detach().clone(), q.grad.clone())
            del h, q
    finally:
        P._split_mode = mode
    print(f"[memory] {layers} layers held for backward: auto {held['auto'] / 2**20:.1f} MiB, never "
          f"{held['never'] / 2**20:.1f} MiB; peak auto {peak['auto'] / 2**20:.1f} MiB, never "
          f"{peak['never'] / 2**20:.1f} MiB", flush=True)
    assert held["auto"] - held["never"] == layers * T * hq * d * 2
    assert torch.equal(outs["auto"][0], outs["never"][0]) and torch.equal(outs["auto"][1], outs["never"][1])
