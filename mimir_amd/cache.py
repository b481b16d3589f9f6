"""Attention against a static KV cache (inference path), MI355X-native.

Mirrors Mimir2's ``Cache`` (src/mimir/model/layers.py:107-115) and
``Attention._attention_with_cache`` (layers.py:134-167): the new keys / values
are written into the cache rows at ``cache_lengths[b] + i``, then each query
attends the cache keys ``j < cache_lengths[b] + S`` (``j <= cache_lengths[b] + i``
when causal).  One C-ABI call (``mimir_prefixlm_cache_attn``) does the cache
update and the attention; GQA is read in place (no repeated K/V heads), the mask
is never materialized, and decode (S = 1) splits the key range over the chip.

bf16 only (the inference dtype); there is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import math
from typing import NamedTuple, Optional

import torch
from torch import Tensor

from . import _capi
from . import prefixlm as P


class Cache(NamedTuple):
    """A static cache layer: keys / values [max_batch, max_seq_len, Hkv, D] (layers.py:107-115)."""
    keys: Tensor
    values: Tensor

    @classmethod
    def create(cls, max_batch_size: int, max_seq_len: int, num_heads: int, head_dim: int, **kwargs):
        return cls(keys=torch.zeros((max_batch_size, max_seq_len, num_heads, head_dim), **kwargs),
                   values=torch.zeros((max_batch_size, max_seq_len, num_heads, head_dim), **kwargs))


def _rows4(name: str, t: Tensor) -> Tensor:
    if t.dim() != 4:
        raise ValueError(f"{name} must be [batch, tokens, heads, head_dim], got shape {tuple(t.shape)}")
    P._check_device_tensor(name, t)
    if t.stride(-1) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.stride(2) % 8 or t.data_ptr() % 16:
        t = t.contiguous()
    return t


def attention_with_cache(query: Tensor, key: Tensor, value: Tensor, cache: Cache, cache_lengths: Tensor,
                         causal: bool, cache_batch_indices: Optional[Tensor] = None,
                         softmax_scale: Optional[float] = None) -> Tensor:
    """``Attention._attention_with_cache`` (layers.py:134-167) for query [B, S, Hq, D] and
    key / value [B, S, Hkv, D]; updates ``cache`` in place and returns [B, S, Hq, D].

    No host synchronisation by default: the key split is sized for the whole cache
    (``cache_len`` positions) instead of the reference's ``kv_len.max().item()``
    (layers.py:143), so decode steps can be captured in a HIP graph.  With
    ``mimir_amd.set_validate_metadata(True)`` it reads the lengths once, as the
    reference does, sizes the split exactly and raises ``IndexError`` where the
    reference's cache write would index past the cache (without validation such
    rows are not written and their keys are ignored).
    """
    if query.dtype != torch.bfloat16:
        raise TypeError(f"KV-cache attention supports bfloat16 tensors only, got {query.dtype}")
    B, S, hq, d = query.shape
    hkv = key.shape[2]
    if key.shape != (B, S, hkv, d) or value.shape != key.shape:
        raise ValueError(f"incompatible query / key / value shapes {tuple(query.shape)}, {tuple(key.shape)}, "
                         f"{tuple(value.shape)}")
    if hq % hkv:
        raise ValueError(f"Query heads {hq} must be divisible by key/value heads {hkv}.")
    ck, cv = cache.keys, cache.values
    if ck.dim() != 4 or ck.shape[2:] != (hkv, d) or cv.shape != ck.shape or ck.dtype != query.dtype:
        raise ValueError(f"cache must be [rows, positions, {hkv}, {d}] {query.dtype}, got {tuple(ck.shape)} {ck.dtype}")
    if ck.stride(-1) != 1 or cv.stride(-1) != 1:
        raise ValueError("cache tensors need a unit head_dim stride")
    q, k, v = _rows4("query", query), _rows4("key", key), _rows4("value", value)
    device = q.device
    # int32 and int64 indices are read as they are (no conversion launch)
    index_dtype = cache_lengths.dtype if cache_lengths.dtype in (torch.int32, torch.int64) else torch.int64
    lens = cache_lengths.to(device=device, dtype=index_dtype).contiguous()
    if lens.shape != (B,):
        raise ValueError(f"cache_lengths must be [{B}], got {tuple(lens.shape)}")
    rows = None
    if cache_batch_indices is not None:
        rows = cache_batch_indices.to(device=device, dtype=index_dtype).contiguous()
        if rows.shape != (B,):
            raise ValueError(f"cache_batch_indices must be [{B}], got {tuple(rows.shape)}")
    L = ck.shape[1]
    max_kv = L
    if B > 0 and P._validate_metadata:  # one host read for all checks (the reference reads kv_len.max() too)
        zero = torch.zeros((), dtype=index_dtype, device=device)
        lmax, lmin, rmin, rmax = torch.stack([lens.max(), lens.min(), rows.min() if rows is not None else zero,
                                              rows.max() if rows is not None else zero]).tolist()
        max_kv = lmax + S
        if lmin < 0:
            raise ValueError(f"cache_lengths must be non-negative, got {lmin}")
        if max_kv > L:
            raise IndexError(f"cache position {max_kv - 1} is out of bounds for a cache of {L} positions")
        if rows is not None and (rmin < 0 or rmax >= ck.shape[0]):
            raise IndexError(f"cache_batch_indices must lie in [0, {ck.shape[0]}), got [{rmin}, {rmax}]")
        if rows is None and B > ck.shape[0]:
            raise IndexError(f"batch of {B} rows for a cache of {ck.shape[0]} rows")
    out = torch.empty((B, S, hq, d), dtype=q.dtype, device=device)
    scale = 1.0 / math.sqrt(d) if softmax_scale is None else float(softmax_scale)
    lib = _capi.load()
    p = _capi.CacheAttnParams(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), ck.data_ptr(), cv.data_ptr(), out.data_ptr(),
        lens.data_ptr(), rows.data_ptr() if rows is not None else None,
        *q.stride()[:3], *k.stride()[:3], *v.stride()[:3], *ck.stride()[:3], *cv.stride()[:3], *out.stride()[:3],
        B, S, L, ck.shape[0], max(max_kv, 1), hq, hkv, d, int(bool(causal)), _capi.DTYPE_BFLOAT16, scale, None, 0,
        int(index_dtype == torch.int64),
    )
    ws_bytes = int(lib.mimir_prefixlm_cache_attn_workspace_bytes(ctypes.byref(p)))
    ws = torch.empty(max(ws_bytes // 4, 4), dtype=torch.float32, device=device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
    _capi.raise_for_status(lib, lib.mimir_prefixlm_cache_attn(ctypes.byref(p), P._stream(device)))
    return out
