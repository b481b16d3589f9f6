"""Pins of the layer oracle (oracle/layer_oracle.py): RoPE, its gradient, the
sigmoid output gate and the composed layer core, on the CPU."""

import math

import pytest
import torch

from oracle import layer_oracle as LO
from oracle.prefixlm_oracle import dense_forward_autograd


def _cos_sin(T, d, base=10000.0, dtype=torch.float32, offset=0):
    """RotaryEmbedding's tables (layers.py:43-59 restated): emb = cat(freqs, freqs)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, d, 2, dtype=torch.float64) / d))
    t = torch.arange(offset, offset + T, dtype=torch.float64)
    emb = torch.cat((torch.outer(t, inv_freq),) * 2, dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def test_rope_identity_at_zero_angle():
    x = torch.randn(5, 3, 16, dtype=torch.bfloat16)
    cos, sin = torch.ones(5, 16), torch.zeros(5, 16)
    assert torch.equal(LO.apply_rotary_pos_emb(x, cos, sin), x)


def test_rope_rotates_pairs_fp64():
    """Each (d, d + D/2) pair turns by its angle: norms kept, +t then -t returns x."""
    x = torch.randn(7, 2, 32, dtype=torch.float64)
    cos, sin = _cos_sin(7, 32, dtype=torch.float64)
    y = LO.apply_rotary_pos_emb(x, cos, sin)
    h = 16
    assert torch.allclose(x[..., :h] ** 2 + x[..., h:] ** 2, y[..., :h] ** 2 + y[..., h:] ** 2, rtol=1e-12, atol=1e-12)
    back = LO.apply_rotary_pos_emb(y, cos, -sin)
    assert torch.allclose(back, x, rtol=1e-12, atol=1e-12)
    # the rotation of pair (x1, x2) by angle a is (x1 cos a - x2 sin a, x2 cos a + x1 sin a)
    a = torch.atan2(sin[:, :h], cos[:, :h]).unsqueeze(1)
    assert torch.allclose(y[..., :h], x[..., :h] * torch.cos(a) - x[..., h:] * torch.sin(a), atol=1e-12)
    assert torch.allclose(y[..., h:], x[..., h:] * torch.cos(a) + x[..., :h] * torch.sin(a), atol=1e-12)


def test_rope_one_rounding_per_op_bf16():
    """bf16 x against fp32 tables: separately rounded fp32 products, one fp32 add, one cast."""
    torch.manual_seed(1)
    x = torch.randn(9, 4, 64, dtype=torch.bfloat16)
    cos, sin = _cos_sin(9, 64, offset=100)
    y = LO.apply_rotary_pos_emb(x, cos, sin)
    xf = x.float().numpy()
    c, s = cos.numpy()[:, None, :], sin.numpy()[:, None, :]
    h = 32
    import numpy as np
    y1 = (xf[..., :h] * c[..., :h]).astype(np.float32) - (xf[..., h:] * s[..., :h]).astype(np.float32)
    y2 = (xf[..., h:] * c[..., h:]).astype(np.float32) + (xf[..., :h] * s[..., h:]).astype(np.float32)
    ref = torch.from_numpy(np.concatenate([y1, y2], axis=-1).astype(np.float32)).to(torch.bfloat16)
    assert torch.equal(y, ref)


def test_rope_grad_is_the_transpose_fp64():
    x = torch.randn(6, 3, 16, dtype=torch.float64)
    g = torch.randn(6, 3, 16, dtype=torch.float64)
    cos, sin = _cos_sin(6, 16, dtype=torch.float64, offset=7)
    lhs = (LO.apply_rotary_pos_emb(x, cos, sin) * g).sum()
    rhs = (x * LO.rope_grad(x, cos, sin, g)).sum()
    assert math.isclose(lhs.item(), rhs.item(), rel_tol=1e-12, abs_tol=1e-12)
    xx = x.clone().requires_grad_(True)
    assert torch.autograd.gradcheck(lambda t: LO.apply_rotary_pos_emb(t, cos, sin), (xx,))


def test_rope_grad_rounding_bf16():
    """Autograd rounds each contribution to bf16 before summing them in bf16."""
    torch.manual_seed(2)
    x = torch.randn(5, 2, 32, dtype=torch.bfloat16)
    g = torch.randn(5, 2, 32, dtype=torch.bfloat16)
    cos, sin = _cos_sin(5, 32, offset=33)
    gx = LO.rope_grad(x, cos, sin, g)
    h = 16
    gf, c, s = g.float(), cos[:, None, :], sin[:, None, :]
    bf = lambda t: t.to(torch.bfloat16).float()
    d1 = bf(bf(gf[..., :h] * c[..., :h]) + bf(gf[..., h:] * s[..., h:]))
    d2 = bf(bf(gf[..., h:] * c[..., h:]) - bf(gf[..., :h] * s[..., :h]))
    assert torch.equal(gx.float(), torch.cat([d1, d2], dim=-1))


def test_gate_closed_forms_fp64():
    gate = torch.randn(4, 2, 8, dtype=torch.float64)
    attn = torch.randn(4, 2, 8, dtype=torch.float64)
    dy = torch.randn(4, 2, 8, dtype=torch.float64)
    assert torch.equal(LO.gate_forward(torch.zeros_like(gate), attn), attn / 2)
    s = 1.0 / (1.0 + torch.exp(-gate))
    assert torch.allclose(LO.gate_forward(gate, attn), s * attn, rtol=1e-14)
    dg, da = LO.gate_backward(gate, attn, dy)
    assert torch.allclose(dg, dy * attn * s * (1 - s), rtol=1e-12, atol=1e-14)
    assert torch.allclose(da, dy * s, rtol=1e-14)


@pytest.mark.parametrize("with_rope", [True, False])
def test_gated_attention_chain_fp64(with_rope):
    """The composed oracle equals fp64 autograd through split -> RoPE -> attention -> gate."""
    torch.manual_seed(3)
    hq, hkv, d = 4, 2, 16
    lens, prefixes = [7, 5], [3, 0]
    T = sum(lens)
    cu = torch.tensor([0, 7, 12], dtype=torch.int32)
    pl = torch.tensor(prefixes, dtype=torch.int32)
    cl = torch.tensor([l - p for l, p in zip(lens, prefixes)], dtype=torch.int32)
    gqkv = torch.randn(T, (2 * hq + 2 * hkv) * d, dtype=torch.float64)
    dy = torch.randn(T, hq, d, dtype=torch.float64)
    cos, sin = _cos_sin(T, d, dtype=torch.float64) if with_rope else (None, None)
    y, dg = LO.gated_attention(gqkv, cos, sin, hq, hkv, False, pl, cl, cu, T, 2, grad_y=dy)

    g = gqkv.clone().requires_grad_(True)
    gate, q, k, v = LO.split_gqkv(g, hq, hkv)
    if with_rope:
        q, k = LO.apply_rotary_pos_emb(q, cos, sin), LO.apply_rotary_pos_emb(k, cos, sin)
    attn = dense_forward_autograd(q, k, v, False, pl, cl, cu, T, 2)
    y_ref = torch.sigmoid(gate) * attn
    (dg_ref,) = torch.autograd.grad(y_ref, g, dy)
    assert torch.allclose(y, y_ref, rtol=1e-10, atol=1e-12)
    assert torch.allclose(dg.reshape(T, -1), dg_ref, rtol=1e-9, atol=1e-11)


def test_cache_attention_empty_cache_is_prefixlm():
    """cache_lengths = 0: causal == prefix-LM with p = 0, bidirectional == p = n (per batch row)."""
    from oracle.prefixlm_oracle import dense_forward
    torch.manual_seed(4)
    B, S, hq, hkv, d, L = 3, 9, 4, 2, 16, 20
    q = torch.randn(B, S, hq, d, dtype=torch.float64)
    k = torch.randn(B, S, hkv, d, dtype=torch.float64)
    v = torch.randn(B, S, hkv, d, dtype=torch.float64)
    for causal in (True, False):
        ck, cv = torch.zeros(B, L, hkv, d, dtype=torch.float64), torch.zeros(B, L, hkv, d, dtype=torch.float64)
        out = LO.attention_with_cache(q, k, v, ck, cv, torch.zeros(B, dtype=torch.int64), causal)
        cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32)
        p = 0 if causal else S
        pl = torch.full((B,), p, dtype=torch.int32)
        cl = torch.full((B,), S - p, dtype=torch.int32)
        ref = dense_forward(q.reshape(B * S, hq, d), k.reshape(B * S, hkv, d), v.reshape(B * S, hkv, d), False,
                            pl, cl, cu, B * S, B)
        assert torch.allclose(out.reshape(B * S, hq, d), ref, rtol=1e-10, atol=1e-12)
        assert torch.equal(ck[:, :S], k) and torch.equal(cv[:, :S], v) and not ck[:, S:].any()


@pytest.mark.parametrize("causal", [True, False])
def test_cache_attention_brute_force(causal):
    """Non-empty caches, chunked prefill and decode, GQA, batch_indices, against fp64 loops."""
    torch.manual_seed(5)
    B, hq, hkv, d, L = 3, 4, 2, 8, 24
    for S in (1, 5):
        q = torch.randn(B, S, hq, d, dtype=torch.float64)
        k = torch.randn(B, S, hkv, d, dtype=torch.float64)
        v = torch.randn(B, S, hkv, d, dtype=torch.float64)
        ck, cv = torch.randn(5, L, hkv, d, dtype=torch.float64), torch.randn(5, L, hkv, d, dtype=torch.float64)
        ck0, cv0 = ck.clone(), cv.clone()
        lens = torch.tensor([0, 7, 13])
        rows = torch.tensor([4, 0, 2])
        out = LO.attention_with_cache(q, k, v, ck, cv, lens, causal, rows)
        scale = d ** -0.5
        for b in range(B):
            r, c = int(rows[b]), int(lens[b])
            keys, vals = ck0[r].clone(), cv0[r].clone()
            keys[c:c + S], vals[c:c + S] = k[b], v[b]
            assert torch.equal(ck[r, :c + S], keys[:c + S])
            for i in range(S):
                n = c + i + 1 if causal else c + S
                for h in range(hq):
                    kk, vv = keys[:n, h // (hq // hkv)], vals[:n, h // (hq // hkv)]
                    w = torch.softmax((kk @ q[b, i, h]) * scale, dim=0)
                    assert torch.allclose(out[b, i, h], w @ vv, rtol=1e-10, atol=1e-12)
