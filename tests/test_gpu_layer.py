"""GPU parity of the fused layer core (mimir_amd.layer) against the CPU layer oracle.

* RoPE kernel: bit-exact against the oracle's restatement of layers.py:24-40
  (forward: one fp32 rounding per operation and one cast; gradient: autograd's
  two element-type roundings and their sum), bf16 and fp32, strided and in place.
* Gated attention (split -> RoPE -> prefix-LM attention -> sigmoid gate), forward
  and gqkv gradient against the oracle chain.  Tolerances (max-abs, the
  operator's contract): bf16 y <= 2e-2, gqkv gradient <= 5e-2; fp32 y <= 1e-5,
  gradient <= 1e-4.  The gated forward leaves the attention output itself
  bitwise equal to the ungated call's.
"""

import pytest
import torch

from mimir_amd import layer as L
from mimir_amd import prefixlm as P
from mimir_amd.workloads import make_case
from oracle import layer_oracle as LO

pytestmark = pytest.mark.gpu

TOL = {torch.bfloat16: dict(y=2e-2, grad=5e-2), torch.float32: dict(y=1e-5, grad=1e-4)}


def _cos_sin(positions, d, base=10000.0):
    inv_freq = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat((torch.outer(positions.float(), inv_freq),) * 2, dim=-1)
    return emb.cos(), emb.sin()


def _positions(seq_lens, T):
    pos = torch.zeros(T, dtype=torch.int64)
    off = 0
    for n in seq_lens:
        pos[off:off + n] = torch.arange(n)
        off += n
    return pos


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.bfloat16, 64), (torch.float32, 64)])
@pytest.mark.parametrize("inverse", [False, True])
def test_rope_bitwise(device, dtype, d, inverse):
    gen = torch.Generator().manual_seed(11)
    T, H = 300, 12
    big = torch.randn(T, H, d, generator=gen).to(dtype)
    x = big[:, 3:8]                      # a strided head slice, like q of the fused projection
    cos, sin = _cos_sin(torch.arange(T) * 7 % 1999, d)
    if inverse:  # x plays the upstream gradient; the map is linear, so the primal point is immaterial
        ref = LO.rope_grad(torch.zeros_like(x), cos, sin, x)
    else:
        ref = LO.apply_rotary_pos_emb(x, cos, sin)
    xd = x.to(device)
    got = L.rope(xd, cos.to(device), sin.to(device), inverse=inverse)
    torch.cuda.synchronize()
    print(f"[rope] {dtype} d={d} inverse={inverse} mismatches={(got.cpu() != ref).sum().item()}", flush=True)
    assert torch.equal(got.cpu(), ref)
    # in place on the strided view
    bigd = big.to(device)
    L.rope(bigd[:, 3:8], cos.to(device), sin.to(device), inverse=inverse, out=bigd[:, 3:8])
    torch.cuda.synchronize()
    assert torch.equal(bigd[:, 3:8].cpu(), ref)
    assert torch.equal(bigd[:, :3].cpu(), big[:, :3]) and torch.equal(bigd[:, 8:].cpu(), big[:, 8:])


CASES = [
    # seq_lens, prefixes, hq, hkv, d, dtype, rope
    ([190, 64, 3], [64, 64, 0], 8, 2, 128, torch.bfloat16, True),
    ([130, 257], [0, 257], 4, 4, 64, torch.bfloat16, True),
    ([200], [77], 4, 1, 128, torch.bfloat16, False),
    ([70, 33], [20, 33], 4, 2, 64, torch.float32, True),
]


@pytest.mark.parametrize("idx", range(len(CASES)))
def test_gated_attention_matches_oracle(device, idx):
    seq_lens, prefixes, hq, hkv, d, dtype, with_rope = CASES[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, dtype=dtype, seed=20 + idx)
    T = case.T
    gen = torch.Generator().manual_seed(40 + idx)
    gqkv = torch.randn(T, (2 * hq + 2 * hkv) * d, generator=gen).to(dtype)
    dy = torch.randn(T, hq, d, generator=gen).to(dtype)
    cos, sin = _cos_sin(_positions(seq_lens, T), d) if with_rope else (None, None)
    y_ref, dg_ref = LO.gated_attention(gqkv, cos, sin, hq, hkv, False, *case.oracle_args(), grad_y=dy)

    c = case.to(device)
    g = gqkv.to(device).requires_grad_(True)
    cs = None if cos is None else (cos.to(device), sin.to(device))
    y = L.gated_attention(g, cs, hq, hkv, False, prefix_lens=c.prefix_lens, causal_lens=c.causal_lens,
                          cu_seqlens=c.cu_seqlens, total_seqlen=c.total_seqlen, numseqs=c.numseqs,
                          max_seqlen_all=c.max_seqlen_all)
    y.backward(dy.to(device).reshape(T, hq * d))
    torch.cuda.synchronize()
    tol = TOL[dtype]
    ey = (y.detach().float().cpu().reshape(T, hq, d) - y_ref.float()).abs().max().item()
    eg = (g.grad.float().cpu().reshape(T, -1, d) - dg_ref.float()).abs().max().item()
    print(f"[gated] {dtype} d={d} seqs={seq_lens} rope={with_rope} err y={ey:.3g} dgqkv={eg:.3g}", flush=True)
    assert ey <= tol["y"]
    assert eg <= tol["grad"]


def test_gate_leaves_attention_output_unchanged(device):
    """The gated launch writes the same O (bitwise) as the plain launch, plus y."""
    hq, hkv, d = 8, 2, 128
    case = make_case([190, 64, 3], [64, 64, 0], hq, hkv, d, dtype=torch.bfloat16, seed=5)
    c = case.to(device)
    gate = torch.randn(case.T, hq, d, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).to(device)
    lib = P._capi.load()
    import ctypes
    args = (c.q, c.k, c.v, False, c.prefix_lens, c.causal_lens, c.cu_seqlens, c.total_seqlen, c.numseqs,
            c.max_seqlen_all, d ** -0.5)
    p0, o0, l0, k0 = P.prepare_fwd(*args)
    P._capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p0), P._stream(c.q.device)))
    y = torch.empty_like(o0)
    p1, o1, l1, k1 = P.prepare_fwd(*args, gate=gate, gated_out=y)
    P._capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p1), P._stream(c.q.device)))
    torch.cuda.synchronize()
    assert torch.equal(o0, o1) and torch.equal(l0, l1)
    y_ref = LO.gate_forward(gate.cpu(), o0.cpu())
    # same rounding as torch.sigmoid(gate) * attn in bf16; sigmoid's last fp32 bit may differ
    diff = (y.cpu().float() - y_ref.float()).abs()
    print(f"[gate store] max diff vs torch bf16 gate: {diff.max().item():.3g}, "
          f"mismatching elements {(diff > 0).sum().item()} of {diff.numel()}", flush=True)
    assert diff.max().item() <= 2 ** -7 * y_ref.float().abs().max().item()
    assert (diff > 0).float().mean().item() < 1e-3


FUSED = [
    # seq_lens, prefixes, hq, hkv, d, total_seqlen (None: all)
    ([190, 64, 3], [64, 64, 0], 8, 2, 128, None),
    ([300, 257], [0, 100], 4, 4, 64, None),
    ([300, 500], [50, 100], 8, 2, 128, 300 + 250),  # total_seqlen inside the second sequence
]


@pytest.mark.parametrize("where", [("fwd", "bwd"), ("fwd",), ("bwd",), ()], ids=["fwd+bwd", "fwd", "bwd", "passes"])
@pytest.mark.parametrize("idx", range(len(FUSED)))
def test_fused_rope_matches_separate_passes(device, idx, where, monkeypatch):
    """bf16 RoPE inside the kernels (q rotated as the forward loads it, dQ / dK mapped back in
    the backward's stores), and the layer's merged passes, against the separate per-tensor
    passes: rope(q), rope(k), the attention, and rope's inverse on dQ / dK.  Same operands bit
    for bit, hence the same y, gqkv gradient and rotated-q copy bit for bit."""
    monkeypatch.setattr(L, "_ROPE_IN_KERNELS", frozenset(where))
    seq_lens, prefixes, hq, hkv, d, total = FUSED[idx]
    case = make_case(seq_lens, prefixes, hq, hkv, d, dtype=torch.bfloat16, seed=50 + idx)
    if total is not None:
        case.total_seqlen = torch.tensor(total, dtype=torch.int64)
    T = case.T
    gen = torch.Generator().manual_seed(60 + idx)
    gqkv = torch.randn(T, (2 * hq + 2 * hkv) * d, generator=gen).to(torch.bfloat16).to(device)
    dy = torch.randn(T, hq * d, generator=gen).to(torch.bfloat16).to(device)
    cos, sin = (t.to(device) for t in _cos_sin(_positions(seq_lens, T), d))
    c = case.to(device)
    meta = dict(prefix_lens=c.prefix_lens, causal_lens=c.causal_lens, cu_seqlens=c.cu_seqlens,
                total_seqlen=c.total_seqlen, numseqs=c.numseqs, max_seqlen_all=c.max_seqlen_all)

    g1 = gqkv.clone().requires_grad_(True)
    y1 = L.gated_attention(g1, (cos, sin), hq, hkv, False, **meta)
    y1.backward(dy)

    g3 = gqkv.view(T, -1, d)
    rot = g3.clone()
    rot[:, hq:2 * hq] = L.rope(g3[:, hq:2 * hq], cos, sin)
    rot[:, 2 * hq:2 * hq + hkv] = L.rope(g3[:, 2 * hq:2 * hq + hkv], cos, sin)
    g2 = rot.reshape(T, -1).requires_grad_(True)
    y2 = L.gated_attention(g2, None, hq, hkv, False, **meta)
    y2.backward(dy)
    dg2 = g2.grad.view(T, -1, d).clone()
    dg2[:, hq:2 * hq] = L.rope(dg2[:, hq:2 * hq], cos, sin, inverse=True)
    dg2[:, 2 * hq:2 * hq + hkv] = L.rope(dg2[:, 2 * hq:2 * hq + hkv], cos, sin, inverse=True)
    torch.cuda.synchronize()
    dg1 = g1.grad.view(T, -1, d)
    print(f"[fused rope] case{idx} {where} d={d} y mismatches {(y1 != y2).sum().item()}, "
          f"grad mismatches {(dg1 != dg2).sum().item()}", flush=True)
    assert torch.equal(y1, y2)
    assert torch.equal(dg1, dg2)

    # the rotated q the forward writes for the backward: rope(q) on every active row
    q = g3[:, hq:2 * hq]
    q_rope = torch.full((T, hq, d), float("nan"), dtype=torch.bfloat16, device=device)
    k_rope = L.rope(g3[:, 2 * hq:2 * hq + hkv], cos, sin)
    p, o, lse, keep = P.prepare_fwd(q, k_rope, g3[:, 2 * hq + hkv:], False, c.prefix_lens, c.causal_lens,
                                    c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, d ** -0.5,
                                    rope=(cos, sin), q_rope=q_rope)
    import ctypes
    lib = P._capi.load()
    P._capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p), P._stream(device)))
    torch.cuda.synchronize()
    active = int(c.total_seqlen) if total is not None else sum(seq_lens)
    assert torch.equal(q_rope[:active], L.rope(q, cos, sin)[:active])
