"""CPU oracle for the attention layer's core around prefix-LM attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` may import this module, as what the
results of ``mimir_amd.layer`` and ``mimir_amd.cache`` are compared against; the
product path never imports it.

Restates src/mimir/model/layers.py: ``rotate_half`` / ``apply_rotary_pos_emb``
(layers.py:24-40), the gqkv head split (layers.py:182-184), the RoPE calls
(layers.py:186-189) and the sigmoid output gate (layers.py:239), with the
attention itself from ``oracle.prefixlm_oracle``.  The restatements use the same
torch operations in the same dtypes as the reference, so their rounding (and
autograd's, for the gradients) is the reference's; ``tests/test_layer_oracle.py``
pins them:

==========================  =======================================================
function                     pinned by
==========================  =======================================================
``apply_rotary_pos_emb``     cos = 1 / sin = 0 is the identity; fp64 pair rotation
                             preserves pair norms; rotating by +t then -t returns x;
                             explicit pair formula with one fp32 rounding per op
``rope_grad``                fp64 adjointness <R x, g> == <x, R^T g>; finite
                             differences (gradcheck); explicit bf16 rounding of
                             the two autograd contributions
``gate_forward``             sigmoid(0) = 1/2; closed form in fp64
``gate_backward``            fp64 closed forms dgate = dy*attn*s*(1-s), dattn = dy*s
``gated_attention``          fp64 autograd of the composed chain on tiny inputs
``attention_with_cache``     empty cache == the prefix-LM oracle (causal: p = 0;
                             bidirectional: p = n); fp64 brute-force loops for
                             decode and chunked prefill; the cache writes
==========================  =======================================================
"""

from __future__ import annotations

import torch
from torch import Tensor

from oracle.prefixlm_oracle import dense_backward, dense_forward

__all__ = [
    "apply_rotary_pos_emb",
    "attention_with_cache",
    "gate_backward",
    "gate_forward",
    "gated_attention",
    "rope_grad",
    "rotate_half",
    "split_gqkv",
]


def rotate_half(x: Tensor) -> Tensor:
    """layers.py:24-28: cat(-x2, x1) over the two halves of the last dim."""
    x1 = x[..., : x.shape[-1] // 2]
    x2 = x[..., x.shape[-1] // 2:]
    return torch.cat((-x2, x1), dim=-1)


def apply_rotary_pos_emb(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """layers.py:31-40 for x [T, H, D] and cos / sin [T, D] (fp32 math, cast back to x's dtype)."""
    return ((x * cos.unsqueeze(-2)) + (rotate_half(x) * sin.unsqueeze(-2))).to(x.dtype)


def rope_grad(x: Tensor, cos: Tensor, sin: Tensor, grad_y: Tensor) -> Tensor:
    """d/dx of apply_rotary_pos_emb, as torch.autograd forms it in x's dtype."""
    xx = x.detach().clone().requires_grad_(True)
    y = apply_rotary_pos_emb(xx, cos, sin)
    (gx,) = torch.autograd.grad(y, xx, grad_y.to(y.dtype))
    return gx


def gate_forward(gate: Tensor, attn: Tensor) -> Tensor:
    """layers.py:239 (before the head merge): torch.sigmoid(gate) * attn_output."""
    return torch.sigmoid(gate) * attn


def gate_backward(gate: Tensor, attn: Tensor, grad_y: Tensor) -> tuple[Tensor, Tensor]:
    """(d gate, d attn) of gate_forward by torch.autograd in the tensors' dtype."""
    g = gate.detach().clone().requires_grad_(True)
    a = attn.detach().clone().requires_grad_(True)
    y = gate_forward(g, a)
    dg, da = torch.autograd.grad(y, (g, a), grad_y.to(y.dtype))
    return dg, da


def split_gqkv(gqkv: Tensor, hq: int, hkv: int):
    """layers.py:182-184: [T, (2Hq+2Hkv)*D] -> gate, q, k, v heads of [T, H, D]."""
    heads = 2 * hq + 2 * hkv
    T, d = gqkv.shape[0], gqkv.shape[-1] // heads if gqkv.dim() == 2 else gqkv.shape[-1]
    g3 = gqkv.reshape(T, heads, d)
    return g3[:, :hq], g3[:, hq:2 * hq], g3[:, 2 * hq:2 * hq + hkv], g3[:, 2 * hq + hkv:]


def gated_attention(gqkv, cos, sin, hq, hkv, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                    grad_y=None):
    """Forward (and, with ``grad_y``, backward) of the layer core in the reference's dtypes.

    The attention runs in fp32 on the element-type inputs (the oracle of the
    operator, softmax scale 1/sqrt(D)) and its output / gradients are cast to the
    element type, as the operator returns them.  Returns ``y`` [T, Hq, D] and, with ``grad_y``, the
    gqkv gradient [T, 2Hq+2Hkv, D].
    """
    dt = gqkv.dtype
    acc = torch.float32 if dt == torch.bfloat16 else dt  # fp64 inputs (the oracle's own pins) stay fp64
    gate, q, k, v = split_gqkv(gqkv, hq, hkv)
    if cos is not None:
        qr, kr = apply_rotary_pos_emb(q, cos, sin), apply_rotary_pos_emb(k, cos, sin)
    else:
        qr, kr = q, k
    attn32 = dense_forward(qr.to(acc), kr.to(acc), v.to(acc), is_causal, prefix_lens, causal_lens, cu_seqlens,
                           total_seqlen, numseqs)
    attn = attn32.to(dt)
    y = gate_forward(gate, attn)
    if grad_y is None:
        return y
    dgate, dattn = gate_backward(gate, attn, grad_y)
    dq, dk, dv = dense_backward(qr.to(acc), kr.to(acc), v.to(acc), attn32, dattn.to(acc), is_causal, prefix_lens,
                                causal_lens, cu_seqlens, total_seqlen, numseqs)
    dq, dk, dv = dq.to(dt), dk.to(dt), dv.to(dt)
    if cos is not None:
        dq, dk = rope_grad(q, cos, sin, dq), rope_grad(k, cos, sin, dk)
    return y, torch.cat((dgate, dq, dk, dv), dim=1)


def attention_with_cache(query, key, value, cache_keys, cache_values, cache_lengths, causal,
                         cache_batch_indices=None):
    """layers.py:134-167 restated: write key / value into the cache, attend with the
    reference's float mask (finfo.min where not allowed).  Inputs [B, S, H, D]; the
    cache tensors are updated in place; the math runs in fp32 (fp64 stays fp64).
    Returns [B, S, Hq, D] in the query's dtype."""
    batch_size, seqlen = query.shape[:2]
    positions = cache_lengths[:, None] + torch.arange(seqlen, dtype=cache_lengths.dtype)
    rows = torch.arange(batch_size) if cache_batch_indices is None else cache_batch_indices
    batch_idx = rows[:, None]
    cache_keys[batch_idx, positions] = key
    cache_values[batch_idx, positions] = value
    kv_len = cache_lengths + seqlen
    max_kv_len = int(kv_len.max().item())
    keys = cache_keys[rows, :max_kv_len]
    values = cache_values[rows, :max_kv_len]
    hq, hkv = query.shape[2], key.shape[2]
    if hq != hkv:
        keys = keys.repeat_interleave(hq // hkv, dim=2)
        values = values.repeat_interleave(hq // hkv, dim=2)
    acc = torch.float64 if query.dtype == torch.float64 else torch.float32
    q, k, v = query.transpose(1, 2).to(acc), keys.transpose(1, 2).to(acc), values.transpose(1, 2).to(acc)
    key_positions = torch.arange(max_kv_len)
    valid = key_positions[None, :] < kv_len[:, None]
    if causal:
        valid = valid[:, None, :] & (key_positions[None, None, :] <= positions[:, :, None])
    else:
        valid = valid[:, None, :]
    mask = torch.zeros((batch_size, seqlen, max_kv_len), dtype=acc).masked_fill(~valid, torch.finfo(acc).min)
    out = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask[:, None])
    return out.transpose(1, 2).to(query.dtype)
