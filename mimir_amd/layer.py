"""The attention layer's core around the prefix-LM operator, fused for MI355X.

Mimir2's ``Attention.forward`` (src/mimir/model/layers.py:169-253) splits the
fused gqkv projection into gate / q / k / v heads (layers.py:182-184), applies
fp32 RoPE to q and k (layers.py:186-189, ``apply_rotary_pos_emb`` at
layers.py:31-40), runs ``flash_attn_varlen_prefixlm`` (layers.py:223-232) and
gates the result with ``torch.sigmoid(gate) * attn_output`` (layers.py:239)
before ``o_proj``.  :func:`gated_attention` is that block, from the projection
output to the tensor ``o_proj`` consumes:

* the split is free: q / k / v / gate are strided views of gqkv, read in place;
* RoPE (the reference's fp32 math and rounding) takes one ``mimir_prefixlm_rope``
  pass over the adjacent q and k heads of gqkv and one inverse pass, in place,
  over the adjacent dQ / dK heads of the gqkv gradient.  For bf16 the attention
  kernels can do both instead (:func:`set_rope_in_kernels`): q rotated as the
  forward loads it (the kernel also writes the rotated copy the backward
  streams), dQ / dK mapped back in the backward's stores -- bit-identical;
* the gate is applied in the attention kernel's store (bf16), and its backward
  is fused with the delta rows of the attention backward;
* dQ / dK / dV and dgate are written straight into one gqkv-shaped gradient.

There is no CPU fallback: the HIP library must be built and the tensors must be
on a ROCm device.
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _capi
from . import prefixlm as P

_DTYPES = {torch.float32: _capi.DTYPE_FLOAT32, torch.bfloat16: _capi.DTYPE_BFLOAT16}

# Where bf16 RoPE runs: in the attention kernels ("fwd": q rotated as the forward
# loads it; "bwd": dQ / dK mapped back in the backward's stores), or (default) in
# one mimir_prefixlm_rope pass over the adjacent q | k heads and one inverse pass
# over dQ | dK.  Both are bit-identical; on MI355X the separate passes measure
# slightly faster: the kernels then read every fp32 cos / sin row once per
# (head, tile) -- four times the bytes of the bf16 rows they rotate -- at the
# start or end of each workgroup, which costs what the two saved passes do.
_ROPE_IN_KERNELS = frozenset(os.environ.get("MIMIR_LAYER_ROPE_IN_KERNELS", "").replace(" ", "").split(",")) - {""}


def set_rope_in_kernels(where) -> None:
    """Where the bf16 layer applies RoPE: a subset of {"fwd", "bwd"} (empty: separate passes)."""
    global _ROPE_IN_KERNELS
    where = frozenset(where)
    if not where <= {"fwd", "bwd"}:
        raise ValueError(f"RoPE placement must be a subset of {{'fwd', 'bwd'}}, got {sorted(where)}")
    _ROPE_IN_KERNELS = where


def rope(x: Tensor, cos: Tensor, sin: Tensor, *, inverse: bool = False, out: Optional[Tensor] = None) -> Tensor:
    """Rotary position embedding of ``x`` [T, H, D] (rotate-half convention,
    src/mimir/model/layers.py:24-40) with float32 ``cos`` / ``sin`` [T, D].

    ``inverse=True`` applies the gradient of that map instead (x_grad from y_grad).
    ``out`` may be ``x`` itself (in place) or any [T, H, D] view with a unit
    head_dim stride; by default a new tensor is returned.
    """
    P._check_device_tensor("x", x)
    if x.dim() != 3:
        raise ValueError(f"x must be [tokens, heads, head_dim], got shape {tuple(x.shape)}")
    if x.dtype not in _DTYPES:
        raise TypeError(f"RoPE supports float32 and bfloat16 tensors only, got {x.dtype}")
    T, H, d = x.shape
    cos = P.rope_rows(cos, T, d, x.device, "cos")
    sin = P.rope_rows(sin, T, d, x.device, "sin")
    if cos.stride(0) != sin.stride(0):
        sin = sin.contiguous()
        cos = cos.contiguous()
    if out is None:
        out = torch.empty((T, H, d), dtype=x.dtype, device=x.device)
    elif out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must match x in shape and dtype")
    xin = P._kernel_layout(x)
    if P._kernel_layout(out) is not out:
        raise ValueError("out needs a unit head_dim stride and 16-byte aligned rows")
    lib = _capi.load()
    p = _capi.RopeParams(
        xin.data_ptr(), out.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        xin.stride(0), xin.stride(1), out.stride(0), out.stride(1), cos.stride(0),
        T, H, d, _DTYPES[x.dtype], int(bool(inverse)),
    )
    _capi.raise_for_status(lib, lib.mimir_prefixlm_rope(ctypes.byref(p), P._stream(x.device)))
    return out


def _split(gqkv: Tensor, hq: int, hkv: int) -> Tuple[int, int, Tensor, Tensor, Tensor, Tensor, Tensor]:
    heads = 2 * hq + 2 * hkv
    if gqkv.shape[-1] % heads:
        raise ValueError(f"gqkv last dim {gqkv.shape[-1]} is not a multiple of 2*Hq + 2*Hkv = {heads}")
    d = gqkv.shape[-1] // heads
    lead = gqkv.shape[:-1]
    T = 1
    for n in lead:
        T *= n
    if len(lead) > 1 and math.prod(lead[:-1]) != 1:
        raise ValueError("packed attention takes one row of tokens: gqkv must be [T, X] or [1, T, X]")
    g3 = gqkv.reshape(T, heads, d)
    return T, d, g3, g3[:, :hq], g3[:, hq:2 * hq], g3[:, 2 * hq:2 * hq + hkv], g3[:, 2 * hq + hkv:]


class _GatedAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gqkv, cos, sin, hq, hkv, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                numseqs, max_seqlen_all, softmax_scale):
        lib = _capi.load()
        T, d, g3, gate, q, k, v = _split(gqkv, hq, hkv)
        bf16 = gqkv.dtype == torch.bfloat16
        fused = bf16 and cos is not None and "fwd" in _ROPE_IN_KERNELS  # q rotated inside the attention kernel
        q_in = q
        if cos is not None:
            if fused:
                q = torch.empty((T, hq, d), dtype=q.dtype, device=q.device)  # the kernel's rotated copy
                k = rope(k, cos, sin)
            else:
                # q and k are adjacent head ranges of gqkv: one pass rotates both
                qk = rope(g3[:, hq:2 * hq + hkv], cos, sin)
                q, k = qk[:, :hq], qk[:, hq:]
        y = torch.empty((T, hq, d), dtype=gqkv.dtype, device=gqkv.device)
        # bf16: the split decision and, when the kernels split, the low half of the
        # attention output (for the backward's delta row sums)
        lo = P._wants_lo(y)
        out_lo = torch.empty_like(y) if lo else y.new_empty(0)
        flag = torch.empty(1 if bf16 else 0, dtype=torch.int32, device=y.device)
        p, out, lse, keep = P.prepare_fwd(q_in if fused else q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens,
                                          total_seqlen, numseqs, max_seqlen_all, softmax_scale, gate=gate,
                                          gated_out=y, out_lo=out_lo if lo else None, split_flag=flag,
                                          rope=(cos, sin) if fused else None, q_rope=q if fused else None)
        _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p), P._stream(y.device)))
        ctx.save_for_backward(gqkv, q, k, out, lse, out_lo, flag, cos, sin, prefix_lens, causal_lens, cu_seqlens)
        ctx.meta = (hq, hkv, is_causal, total_seqlen, numseqs, max_seqlen_all, softmax_scale)
        return y.reshape(*gqkv.shape[:-1], hq * d)

    @staticmethod
    def backward(ctx, dy):
        lib = _capi.load()
        gqkv, q, k, out, lse, out_lo, flag, cos, sin, prefix_lens, causal_lens, cu_seqlens = ctx.saved_tensors
        hq, hkv, is_causal, total_seqlen, numseqs, max_seqlen_all, softmax_scale = ctx.meta
        T, d, g3, gate, _, _, v = _split(gqkv, hq, hkv)
        dg3 = torch.empty_like(g3)
        dgate, dq, dk, dv = dg3[:, :hq], dg3[:, hq:2 * hq], dg3[:, 2 * hq:2 * hq + hkv], dg3[:, 2 * hq + hkv:]
        dy3 = dy.reshape(T, hq, d)
        fused = gqkv.dtype == torch.bfloat16 and cos is not None and "bwd" in _ROPE_IN_KERNELS
        p, dq, dk, dv, keep = P.prepare_bwd(dy3, q, k, v, out, lse, is_causal, prefix_lens, causal_lens, cu_seqlens,
                                            total_seqlen, numseqs, max_seqlen_all, softmax_scale, gate=gate,
                                            dgate=dgate, dq=dq, dk=dk, dv=dv, out_lo=out_lo, split_flag=flag,
                                            rope=(cos, sin) if fused else None)
        _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd(ctypes.byref(p), P._stream(dg3.device)))
        if cos is not None and not fused:
            dqk = dg3[:, hq:2 * hq + hkv]  # dQ and dK, adjacent: one pass maps both back
            rope(dqk, cos, sin, inverse=True, out=dqk)
        return (dg3.reshape(gqkv.shape),) + (None,) * 12


def gated_attention(
    gqkv: Tensor,
    cos_sin: Optional[Tuple[Tensor, Tensor]],
    num_heads: int,
    num_key_value_heads: int,
    is_causal: bool,
    *,
    prefix_lens: Tensor,
    causal_lens: Tensor,
    cu_seqlens: Tensor,
    total_seqlen,
    numseqs,
    max_seqlen_all,
    softmax_scale: Optional[float] = None,
    **unused_seq_info,
) -> Tensor:
    """``sigmoid(gate) * flash_attn_varlen_prefixlm(rope(q), rope(k), v)`` from the fused projection.

    ``gqkv``: the gqkv projection output, [T, (2*Hq + 2*Hkv) * D] or [1, T, ...], heads
    ordered gate, q, k, v (src/mimir/model/layers.py:182-184).  ``cos_sin``: the
    ``RotaryEmbedding`` output (float32 [T, D] each, or None for no RoPE).  The
    metadata keywords are those of ``flash_attn_varlen_prefixlm``
    (flash_attention_prefixlm_v2.py:286-306); routing-only keys are accepted and
    ignored.  Returns [..., T, Hq * D], the input of ``o_proj`` (layers.py:239-247).
    """
    if gqkv.dtype not in _DTYPES:
        raise TypeError(f"gated attention supports float32 and bfloat16 tensors only, got {gqkv.dtype}")
    P._check_device_tensor("gqkv", gqkv)
    hq, hkv = int(num_heads), int(num_key_value_heads)
    if hq % hkv:
        raise ValueError(f"Query heads {hq} must be divisible by key/value heads {hkv}.")
    d = gqkv.shape[-1] // (2 * hq + 2 * hkv)
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else float(softmax_scale)
    cos, sin = (None, None) if cos_sin is None else cos_sin
    return _GatedAttention.apply(gqkv, cos, sin, hq, hkv, bool(is_causal), prefix_lens, causal_lens, cu_seqlens,
                                 total_seqlen, numseqs, max_seqlen_all, scale)
