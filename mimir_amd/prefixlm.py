"""Drop-in prefix-LM attention for MI355X (gfx950).

:func:`flash_attn_varlen_prefixlm` keeps the exact call signature of the
reference entry point (src/mimir/model/flash_attention_prefixlm_v2.py:286-306,
same keyword set as flash_attention_prefixlm_dispatch.py:80-106), so the Mimir2
``Attention.forward`` call (src/mimir/model/layers.py:223-232) reaches this
backend unchanged.  The work is done by hand-written HIP kernels in
``libmimir_prefixlm.so`` behind a C ABI (include/mimir_prefixlm.h); this module
only validates arguments, allocates outputs with torch's caching allocator and
enqueues the library calls on torch's current stream.  There is no CPU or
PyTorch fallback: tensors that are not on a ROCm device, or a missing library,
raise.

Layers:

* ``torch.ops.mimir_amd.prefixlm_fwd`` / ``prefixlm_bwd`` -- ``torch.library``
  custom ops with fake (meta) implementations, the pattern of
  flash_attention_prefixlm_v2.py:101-162,165-246, so ``torch.compile`` traces
  through without a graph break.
* :class:`PrefixLMAttention` -- the autograd function (v2.py:249-283); it saves
  q, k, v, O and the logsumexp and calls the atomic-free backward.
* :func:`prefixlm_attn_fwd` -- lower-level entry returning ``(O, lse)`` with
  ``lse`` float32 ``[Hq, T]`` (FA varlen layout, v2.py:159-160).
"""

from __future__ import annotations

import ctypes
import math
import os
from typing import Optional

import torch
from torch import Tensor

from . import _capi

__all__ = [
    "PrefixLMAttention",
    "check_metadata",
    "flash_attn_varlen_prefixlm",
    "prefixlm_attn_bwd",
    "prefixlm_attn_fwd",
    "set_split_mode",
    "set_validate_metadata",
]

ROUTING_KEYS = (
    "prefix_cu_seqlens",
    "prefix_idx",
    "causal_idx",
    "active_key_idx",
    "active_cu_seqlens_q",
    "active_cu_seqlens_k",
)

_DTYPES = {torch.float32: _capi.DTYPE_FLOAT32, torch.bfloat16: _capi.DTYPE_BFLOAT16}
_validate_metadata = os.environ.get("MIMIR_PREFIXLM_VALIDATE", "0") not in ("", "0")


def set_validate_metadata(enabled: bool) -> None:
    """Check ``prefix_lens + causal_lens == seq_len <= max_seqlen_all`` on every call.

    The check runs on the device and needs one host synchronisation per call, so
    it is off by default (the FA4 path of the reference does not check either);
    the reference's dense path raises ``ValueError`` for a length mismatch
    (flash_attention_prefixlm_dense.py:54-55) and so does this one when enabled,
    also for a sequence longer than ``max_seqlen_all``.  Without the check such a
    sequence is still computed correctly: the tile lists do not depend on
    ``max_seqlen_all``, and the backward falls back to recomputing dQ when a
    stored score-gradient tile would not fit its region.
    """
    global _validate_metadata
    _validate_metadata = bool(enabled)


_dscore_limit_bytes = int(os.environ.get("MIMIR_PREFIXLM_DSCORE_LIMIT", str(4 << 30)))


def set_dscore_workspace_limit(nbytes: int) -> None:
    """Workspace bytes the backward may spend on stored score gradients.

    With bf16 and head_dim 128 the dK / dV kernel can hand its bf16 dS tiles to
    the dQ kernel, which then computes dQ = dS K without recomputing S and dP.
    The tiles take ``Hq * (T / 32 + numseqs + 1) * ceil(max_seqlen / 32) * 2 KiB``
    (about 1.1 GB for 8 x 2048 tokens and 16 heads); above this limit, or (for
    a region above 1/64 of the device's memory) above half of the device memory
    free at the call (what the driver reports plus torch's cached free blocks),
    the dQ kernel recomputes instead; and if the allocation still fails, the
    backward retries without the tiles.  0 turns the hand-off off.  Default 4 GiB.
    """
    global _dscore_limit_bytes
    if nbytes < 0:
        raise ValueError("the limit is a byte count >= 0")
    _dscore_limit_bytes = int(nbytes)


_key_chunks = os.environ.get("MIMIR_PREFIXLM_KEY_CHUNKS", "1") != "0"


def set_key_chunks(enabled: bool) -> None:
    """Whether the bf16 forward and dQ kernels may cut the key ranges of their heaviest query tiles.

    On a small grid (fewer than 512 query-tile x q-head workgroups, e.g. two
    heads over 24k tokens) the heaviest tiles otherwise run alone at the end;
    with this on, the forward's workspace is sized by
    ``mimir_prefixlm_fwd_workspace_size`` and the backward's asks for the dQ
    parts (``dq_key_chunks``; a few tens of MB each on such grids), and the
    kernels split those tiles' key ranges into parts that are merged in a fixed
    order, so results stay deterministic.  They differ from the uncut kernels
    only by fp32 summation order.  Default on.
    """
    global _key_chunks
    _key_chunks = bool(enabled)


_SPLIT_MODES = {"auto": _capi.SPLIT_AUTO, "always": _capi.SPLIT_ALWAYS, "never": _capi.SPLIT_NEVER}
_split_mode = _SPLIT_MODES[os.environ.get("MIMIR_PREFIXLM_SPLIT", "auto")]


def set_split_mode(mode: str) -> None:
    """Whether the bf16 kernels carry P and dS as two bf16 halves: ``"auto"`` (default), ``"always"``, ``"never"``.

    The bf16 MFMA operands round P (forward O = P V) and dS (backward dQ = dS K,
    dK = dS^T Q) to 8 significant bits.  dQ and dK are sums of cancelling terms
    (every row of dS sums to zero) and delta = rowsum(dO * O) inherits O's
    rounding, so with large key / query entries those roundings dominate the
    gradients' error.  Split, each operand is hi + lo (one more MFMA per product)
    and its rounding no longer reaches the result.  ``"auto"`` splits when
    ``softmax_scale * max|K| > 0.75`` anywhere in the call, decided on the
    device by the kernels themselves (no host synchronisation).
    """
    global _split_mode
    if mode not in _SPLIT_MODES:
        raise ValueError(f"split mode must be one of {sorted(_SPLIT_MODES)}, got {mode!r}")
    _split_mode = _SPLIT_MODES[mode]


def _scalar(x) -> int:
    return int(x.item()) if isinstance(x, Tensor) else int(x)


def _check_device_tensor(name: str, t: Tensor) -> None:
    if t.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(
            f"mimir_amd prefix-LM attention runs on ROCm GPUs only; {name} is on {t.device} "
            "(there is no CPU fallback in this backend)"
        )


def _kernel_layout(t: Tensor) -> Tensor:
    """Unit stride on head_dim, 16-byte aligned rows; copies otherwise."""
    vec = 16 // t.element_size()
    if (
        t.stride(-1) != 1
        or t.stride(0) % vec
        or t.stride(1) % vec
        or t.data_ptr() % 16
        or t.stride(0) < t.shape[-1]
    ):
        t = t.contiguous()
    return t


def _metadata(t: Tensor, device: torch.device, n: int, name: str) -> Tensor:
    if t.dim() != 1 or t.shape[0] < n:
        raise ValueError(f"{name} must be a 1-D tensor with at least {n} entries, got shape {tuple(t.shape)}")
    if t.device != device or t.dtype != torch.int32 or not t.is_contiguous():
        t = t.to(device=device, dtype=torch.int32).contiguous()
    return t


def _geometry(q: Tensor, k: Tensor, v: Tensor):
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k and v must be [tokens, heads, head_dim]")
    if k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError(f"incompatible q/k/v shapes {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise TypeError(f"q, k and v must share one dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if q.dtype not in _DTYPES:
        raise TypeError(f"prefix-LM attention supports float32 and bfloat16 tensors only, got {q.dtype}")
    hq, hkv = q.shape[1], k.shape[1]
    if hq % hkv != 0:
        raise ValueError(f"Query heads {hq} must be divisible by key/value heads {hkv}.")
    return q.shape[0], hq, hkv, q.shape[2]


def _stream(device: torch.device) -> int:
    """The device's current stream, as the raw handle torch's own kernel launches use
    (building a ``torch.cuda.Stream`` for it took ~20 us of host time per call)."""
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None
                                               else torch.cuda.current_device())


def check_metadata(prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor, numseqs,
                   max_seqlen_all=None) -> None:
    """Raise ``ValueError`` like flash_attention_prefixlm_dense.py:54-55 for a bad sequence,
    and for a sequence longer than ``max_seqlen_all`` (when given).

    Runs the library's device-side check and synchronises once.
    """
    lib = _capi.load()
    n = _scalar(numseqs)
    max_all = 0x7FFFFFFF if max_seqlen_all is None else _scalar(max_seqlen_all)
    device = cu_seqlens.device
    _check_device_tensor("cu_seqlens", cu_seqlens)
    pl = _metadata(prefix_lens, device, n, "prefix_lens")
    cl = _metadata(causal_lens, device, n, "causal_lens")
    cu = _metadata(cu_seqlens, device, n + 1, "cu_seqlens")
    bad = torch.empty(2, dtype=torch.int32, device=device)
    status = lib.mimir_prefixlm_check_metadata(pl.data_ptr(), cl.data_ptr(), cu.data_ptr(), n, max_all,
                                               bad.data_ptr(), _stream(device))
    _capi.raise_for_status(lib, status)
    s, why = (int(x) for x in bad.tolist())
    if s >= 0:
        p, c = int(pl[s].item()), int(cl[s].item())
        length = int(cu[s + 1].item()) - int(cu[s].item())
        if why == 2:
            raise ValueError(f"PrefixLM sequence {s} has length {length} > max_seqlen_all {max_all}")
        raise ValueError(f"Bad PrefixLM lengths for sequence {s}: {p} + {c} != {length}")


def rope_rows(t: Tensor, T: int, d: int, device, name: str) -> Tensor:
    """A RoPE table (``cos`` or ``sin``) as float32 rows [T, D] on ``device`` with a
    unit column stride and 16-byte aligned rows (copied only if needed)."""
    t = t.reshape(-1, t.shape[-1])
    if t.shape != (T, d):
        raise ValueError(f"{name} must hold one [head_dim] row per token: expected {(T, d)}, got {tuple(t.shape)}")
    if t.device != device or t.dtype != torch.float32 or t.stride(-1) != 1 or t.stride(0) % 4 or t.data_ptr() % 16:
        t = t.to(device=device, dtype=torch.float32).contiguous()
    return t


def _set_rope(p, rope, T: int, d: int, device) -> tuple:
    """Point the params' RoPE tables at ``rope`` = (cos, sin); returns the tensors to keep alive."""
    cos, sin = (rope_rows(t, T, d, device, name) for t, name in zip(rope, ("cos", "sin")))
    if cos.stride(0) != sin.stride(0):
        cos, sin = cos.contiguous(), sin.contiguous()
    p.rope_cos, p.rope_sin, p.rope_stride_token = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
    return cos, sin


def prepare_fwd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs, max_seqlen_all,
                softmax_scale, gate=None, gated_out=None, out_lo=None, split_mode=None, split_flag=None, rope=None,
                q_rope=None):
    """Validate, allocate O / lse and fill the C parameter struct of the forward.

    Returns ``(params, out, lse, keep)``; ``keep`` holds every tensor the struct
    points to and must outlive the launch.  With ``gate`` ([T, Hq, D], the
    sigmoid output gate of src/mimir/model/layers.py:239) the launch also writes
    ``gated_out`` (same shape; allocated by the caller, may be a strided view).
    With ``out_lo`` (bf16 [T, Hq, D], caller-allocated) it also writes the low
    half of the output, round(O - round(O)), which the backward's row sums use.
    ``split_mode`` is a ``_capi.SPLIT_*`` mode (default: :func:`set_split_mode`);
    with ``split_flag`` (int32 [1], caller-allocated) the launch records its split
    decision there and writes ``out_lo`` only when it splits.
    With ``rope`` = (cos, sin) (float32 [T, D], bf16 only) the kernel rotates q as
    it loads it (``k`` must already be rotated) and, given ``q_rope`` ([T, Hq, D],
    caller-allocated), writes the rotated q there for the backward.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        _check_device_tensor(name, t)
    T, hq, hkv, d = _geometry(q, k, v)
    n = _scalar(numseqs)
    device = q.device
    pl = _metadata(prefix_lens, device, n, "prefix_lens")
    cl = _metadata(causal_lens, device, n, "causal_lens")
    cu = _metadata(cu_seqlens, device, n + 1, "cu_seqlens")
    max_all = _scalar(max_seqlen_all)
    if _validate_metadata:
        check_metadata(pl, cl, cu, n, max_all)
    q, k, v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
    out = torch.empty((T, hq, d), dtype=q.dtype, device=device)
    lse = torch.empty((hq, T), dtype=torch.float32, device=device)
    p = _capi.FwdParams(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(),
        pl.data_ptr(), cl.data_ptr(), cu.data_ptr(),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), lse.stride(0),
        T, hq, hkv, d, n, _scalar(total_seqlen), max_all, int(bool(is_causal)),
        _DTYPES[q.dtype], float(softmax_scale), 0, 0,
    )
    lib = _capi.load()
    ws_bytes = int(lib.mimir_prefixlm_fwd_workspace_size(ctypes.byref(p)) if _key_chunks
                   else lib.mimir_prefixlm_fwd_workspace_bytes(T, n, max_all))
    ws = torch.empty(max(ws_bytes // 4, 4), dtype=torch.float32, device=device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
    p.split_mode = _split_mode if split_mode is None else int(split_mode)
    keep = (q, k, v, pl, cl, cu, ws)
    if split_flag is not None and split_flag.numel() > 0:
        p.split_flag = split_flag.data_ptr()
        keep = keep + (split_flag,)
    if gate is not None:
        gate = _gate_operand("gate", gate, (T, hq, d), q.dtype)
        _gate_operand("gated_out", gated_out, (T, hq, d), q.dtype, copy=False)
        p.gate, p.gate_stride_token, p.gate_stride_head = gate.data_ptr(), gate.stride(0), gate.stride(1)
        p.gated_out = gated_out.data_ptr()
        p.gated_out_stride_token, p.gated_out_stride_head = gated_out.stride(0), gated_out.stride(1)
        keep = keep + (gate, gated_out)
    if out_lo is not None:
        _gate_operand("out_lo", out_lo, (T, hq, d), q.dtype, copy=False)
        p.out_lo, p.out_lo_stride_token, p.out_lo_stride_head = out_lo.data_ptr(), out_lo.stride(0), out_lo.stride(1)
        keep = keep + (out_lo,)
    if rope is not None:
        keep = keep + _set_rope(p, rope, T, d, device)
        if q_rope is not None:
            _gate_operand("q_rope", q_rope, (T, hq, d), q.dtype, copy=False)
            p.q_rope, p.q_rope_stride_token, p.q_rope_stride_head = q_rope.data_ptr(), q_rope.stride(0), q_rope.stride(1)
            keep = keep + (q_rope,)
    return p, out, lse, keep


def _gate_operand(name: str, t, shape, dtype, copy: bool = True) -> Tensor:
    """A gate-side tensor: [T, Hq, D] of the attention's dtype on its device.  Inputs
    are re-laid out if the kernels cannot read them in place; outputs must already
    have a unit head_dim stride and 16-byte aligned rows."""
    if t is None:
        raise ValueError(f"{name} is required with a gate")
    _check_device_tensor(name, t)
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    laid = _kernel_layout(t)
    if laid is not t and not copy:
        raise ValueError(f"{name} needs a unit head_dim stride and 16-byte aligned rows")
    return laid


def _wants_lo(q: Tensor) -> bool:
    """Whether a bf16 forward keeps its output's low half for the backward.

    With split mode "auto" (the default) or "always" the low half O_lo = round(O -
    round(O)) is allocated for every bf16 call and saved for the backward: one more
    [T, Hq, D] bf16 tensor per attention call held from forward to backward (64 MiB
    at 8 x 2048 tokens, 16 heads, head_dim 128), written only when the kernels split.
    "never" skips it.  The mode is read when the call is made (under torch.compile,
    when it is traced).
    """
    return q.dtype == torch.bfloat16 and _split_mode != _capi.SPLIT_NEVER


def _fwd_impl(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs, max_seqlen_all,
              softmax_scale):
    lib = _capi.load()
    # bf16: the split decision and, when it splits, the output's low half (for the
    # backward's delta = rowsum(dO * O)); float32 needs neither
    lo = _wants_lo(q)
    out_lo = torch.empty(q.shape, dtype=q.dtype, device=q.device) if lo else q.new_empty(0)
    flag = torch.empty(1 if q.dtype == torch.bfloat16 else 0, dtype=torch.int32, device=q.device)
    p, out, lse, keep = prepare_fwd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                                    numseqs, max_seqlen_all, softmax_scale, out_lo=out_lo if lo else None,
                                    split_flag=flag)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(p), _stream(out.device)))
    return out, lse, out_lo, flag


def prepare_bwd(dout, q, k, v, out, lse, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                max_seqlen_all, softmax_scale, gate=None, dgate=None, dq=None, dk=None, dv=None, out_lo=None,
                split_mode=None, split_flag=None, rope=None):
    """Validate, allocate dQ / dK / dV and the workspace, fill the backward struct.

    Returns ``(params, dq, dk, dv, keep)``.  With ``gate``, ``dout`` is the
    gradient of the gated output and ``out`` the ungated attention output; the
    launch writes ``dgate`` (caller-allocated).  ``dq`` / ``dk`` / ``dv`` may be
    given as (strided) output views, e.g. slices of a fused gqkv gradient.
    ``out_lo`` is the forward's low output half (bf16), ``split_mode`` a
    ``_capi.SPLIT_*`` mode (default: :func:`set_split_mode`), ``split_flag`` the
    forward's recorded split decision (then followed instead of scanning K).
    With ``rope`` = (cos, sin) (bf16 only), ``q`` / ``k`` are the rotated operands
    the forward used and dQ / dK come back as gradients of the unrotated q / k.

    The workspace holds the score-gradient hand-off region when it fits the
    limit (:func:`set_dscore_workspace_limit`); if that allocation runs out of
    device memory the backward falls back to recomputing dQ with the small
    workspace instead of failing.
    """
    lib = _capi.load()
    for name, t in (("q", q), ("k", k), ("v", v), ("out", out), ("dout", dout)):
        _check_device_tensor(name, t)
    T, hq, hkv, d = _geometry(q, k, v)
    n = _scalar(numseqs)
    device = q.device
    pl = _metadata(prefix_lens, device, n, "prefix_lens")
    cl = _metadata(causal_lens, device, n, "causal_lens")
    cu = _metadata(cu_seqlens, device, n + 1, "cu_seqlens")
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    q, k, v = _kernel_layout(q), _kernel_layout(k), _kernel_layout(v)
    out, dout = _kernel_layout(out), _kernel_layout(dout)
    lse = lse.contiguous()
    dq = torch.empty((T, hq, d), dtype=q.dtype, device=device) if dq is None else _gate_operand(
        "dq", dq, (T, hq, d), q.dtype, copy=False)
    dk = torch.empty((T, hkv, d), dtype=q.dtype, device=device) if dk is None else _gate_operand(
        "dk", dk, (T, hkv, d), q.dtype, copy=False)
    dv = torch.empty((T, hkv, d), dtype=q.dtype, device=device) if dv is None else _gate_operand(
        "dv", dv, (T, hkv, d), q.dtype, copy=False)
    gate_keep = ()
    if gate is not None:
        gate = _gate_operand("gate", gate, (T, hq, d), q.dtype)
        _gate_operand("dgate", dgate, (T, hq, d), q.dtype, copy=False)
        gate_keep = (gate, dgate)
    p = _capi.BwdParams(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), dout.data_ptr(), lse.data_ptr(),
        dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
        pl.data_ptr(), cl.data_ptr(), cu.data_ptr(),
        q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        out.stride(0), out.stride(1), dout.stride(0), dout.stride(1),
        dq.stride(0), dq.stride(1), dk.stride(0), dk.stride(1), dv.stride(0), dv.stride(1),
        lse.stride(0),
        T, hq, hkv, d, n, _scalar(total_seqlen), _scalar(max_seqlen_all), int(bool(is_causal)),
        _DTYPES[q.dtype], float(softmax_scale), 0, 0,
    )
    if gate is not None:
        p.gate, p.gate_stride_token, p.gate_stride_head = gate.data_ptr(), gate.stride(0), gate.stride(1)
        p.dgate, p.dgate_stride_token, p.dgate_stride_head = dgate.data_ptr(), dgate.stride(0), dgate.stride(1)
    if out_lo is not None and out_lo.numel() > 0:
        out_lo = _gate_operand("out_lo", out_lo, (T, hq, d), q.dtype)
        p.out_lo, p.out_lo_stride_token, p.out_lo_stride_head = out_lo.data_ptr(), out_lo.stride(0), out_lo.stride(1)
        gate_keep = gate_keep + (out_lo,)
    p.split_mode = _split_mode if split_mode is None else int(split_mode)
    if split_flag is not None and split_flag.numel() > 0:
        p.split_flag = split_flag.data_ptr()
        gate_keep = gate_keep + (split_flag,)
    if rope is not None:
        gate_keep = gate_keep + _set_rope(p, rope, T, d, device)
    p.dscore_limit_bytes = _dscore_limit_bytes
    p.dq_key_chunks = int(_key_chunks)
    region = int(lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p))) if _dscore_limit_bytes > 0 else 0
    if region > _total_device_bytes(device) // 64:  # a large region: keep it to half of what is free
        p.dscore_limit_bytes = min(_dscore_limit_bytes, _free_device_bytes(device) // 2)
    ws_bytes = int(lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p)))
    try:
        ws = torch.empty(max(ws_bytes // 4, 4), dtype=torch.float32, device=device)
    except torch.cuda.OutOfMemoryError:
        if int(lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p))) == 0:
            raise
        # no room for the score-gradient tiles: the recomputing dQ needs none
        p.dscore_limit_bytes = 0
        ws_bytes = int(lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p)))
        ws = torch.empty(max(ws_bytes // 4, 4), dtype=torch.float32, device=device)
    p.workspace, p.workspace_bytes = ws.data_ptr(), ws_bytes
    return p, dq, dk, dv, (q, k, v, out, dout, lse, pl, cl, cu, ws) + gate_keep


_total_bytes = {}


def _total_device_bytes(device) -> int:
    """The device's memory size (cached per device)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _total_bytes:
        _total_bytes[idx] = int(torch.cuda.get_device_properties(idx).total_memory)
    return _total_bytes[idx]


def _free_device_bytes(device) -> int:
    """Device memory an allocation can still get: free in the driver plus torch's cached free blocks.
    (A few hundred microseconds of host time: asked only for regions above 1/64 of the device.)"""
    free, _total = torch.cuda.mem_get_info(device)
    return int(free) + int(torch.cuda.memory_reserved(device)) - int(torch.cuda.memory_allocated(device))


def _bwd_impl(dout, q, k, v, out, lse, out_lo, split_flag, is_causal, prefix_lens, causal_lens, cu_seqlens,
              total_seqlen, numseqs, max_seqlen_all, softmax_scale):
    lib = _capi.load()
    p, dq, dk, dv, keep = prepare_bwd(dout, q, k, v, out, lse, is_causal, prefix_lens, causal_lens, cu_seqlens,
                                      total_seqlen, numseqs, max_seqlen_all, softmax_scale, out_lo=out_lo,
                                      split_flag=split_flag)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_bwd(ctypes.byref(p), _stream(dq.device)))
    return dq, dk, dv


@torch.library.custom_op("mimir_amd::prefixlm_fwd", mutates_args=())
def _prefixlm_fwd_op(
    q: Tensor, k: Tensor, v: Tensor, is_causal: bool,
    prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
    total_seqlen: Tensor, numseqs: Tensor, max_seqlen_all: Tensor, softmax_scale: float,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """(O, lse, O_lo, split_flag): for bf16 the low output half (written only when the
    kernels split P; empty with split mode "never") and the recorded split decision;
    both empty for float32."""
    return _fwd_impl(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                     max_seqlen_all, softmax_scale)


@_prefixlm_fwd_op.register_fake
def _(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs, max_seqlen_all,
      softmax_scale):
    cf = torch.contiguous_format
    lo = torch.empty_like(q, memory_format=cf) if _wants_lo(q) else q.new_empty(0)
    flag = q.new_empty(1 if q.dtype == torch.bfloat16 else 0, dtype=torch.int32)
    return (torch.empty_like(q, memory_format=cf), q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32), lo,
            flag)


@torch.library.custom_op("mimir_amd::prefixlm_bwd", mutates_args=())
def _prefixlm_bwd_op(
    dout: Tensor, q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, out_lo: Tensor, split_flag: Tensor,
    is_causal: bool, prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
    total_seqlen: Tensor, numseqs: Tensor, max_seqlen_all: Tensor, softmax_scale: float,
) -> tuple[Tensor, Tensor, Tensor]:
    """(dQ, dK, dV); an empty ``out_lo`` means delta from ``out`` alone, an empty
    ``split_flag`` that the backward makes its own split decision."""
    return _bwd_impl(dout, q, k, v, out, lse, out_lo, split_flag, is_causal, prefix_lens, causal_lens, cu_seqlens,
                     total_seqlen, numseqs, max_seqlen_all, softmax_scale)


@_prefixlm_bwd_op.register_fake
def _(dout, q, k, v, out, lse, out_lo, split_flag, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
      numseqs, max_seqlen_all, softmax_scale):
    cf = torch.contiguous_format
    return (torch.empty_like(q, memory_format=cf), torch.empty_like(k, memory_format=cf),
            torch.empty_like(v, memory_format=cf))


def _direct(q: Tensor) -> bool:
    """Whether a call may run the ops' bodies directly: eager, with plain tensors (no
    torch.compile, no tracing or fake-tensor mode, which must see the custom ops)."""
    return (type(q) is Tensor and not torch.compiler.is_compiling()
            and torch._C._len_torch_dispatch_stack() == 0)


def _cpu_scalar(x) -> Tensor:
    if isinstance(x, Tensor):
        return x if x.device.type == "cpu" else x.cpu()
    return torch.tensor(int(x), dtype=torch.int64)


class PrefixLMAttention(torch.autograd.Function):
    """Autograd function over the two custom ops (flash_attention_prefixlm_v2.py:249-283).

    Under torch.compile the ops are what the graph records; run eagerly it calls
    their bodies directly, which skips ~50 us of custom-op dispatch per call (at
    Mimir2's XXS shape the GPU work of a step is ~0.24 ms, so that host time
    showed)."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                max_seqlen_all, softmax_scale):
        fwd = _fwd_impl if _direct(q) else _prefixlm_fwd_op
        out, lse, out_lo, flag = fwd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                                     numseqs, max_seqlen_all, softmax_scale)
        ctx.save_for_backward(q, k, v, out, lse, out_lo, flag, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                              numseqs, max_seqlen_all)
        ctx.mark_non_differentiable(lse)
        ctx.is_causal = bool(is_causal)
        ctx.softmax_scale = float(softmax_scale)
        return out, lse

    @staticmethod
    def backward(ctx, dout, dlse):
        (q, k, v, out, lse, out_lo, flag, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
         max_seqlen_all) = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        bwd = _bwd_impl if _direct(q) else _prefixlm_bwd_op
        dq, dk, dv = bwd(dout, q, k, v, out, lse, out_lo, flag, ctx.is_causal, prefix_lens, causal_lens,
                         cu_seqlens, total_seqlen, numseqs, max_seqlen_all, ctx.softmax_scale)
        return dq, dk, dv, None, None, None, None, None, None, None, None


def prefixlm_attn_fwd(
    q: Tensor, k: Tensor, v: Tensor, is_causal: bool,
    prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
    total_seqlen, numseqs, max_seqlen_all, softmax_scale: Optional[float] = None,
) -> tuple[Tensor, Tensor]:
    """Differentiable prefix-LM attention returning ``(O, lse)``.

    ``lse`` is float32 ``[Hq, T]``: natural log of the softmax denominator with
    the scale included; rows outside every sequence or at/after
    ``total_seqlen`` hold ``-inf`` (and O holds 0).  The gradient flows through
    O only (``lse`` is treated as a non-differentiable auxiliary output).
    """
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else float(softmax_scale)
    return PrefixLMAttention.apply(q, k, v, bool(is_causal), prefix_lens, causal_lens, cu_seqlens,
                                   _cpu_scalar(total_seqlen), _cpu_scalar(numseqs), _cpu_scalar(max_seqlen_all),
                                   scale)


def prefixlm_attn_bwd(
    dout: Tensor, q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, is_causal: bool,
    prefix_lens: Tensor, causal_lens: Tensor, cu_seqlens: Tensor,
    total_seqlen, numseqs, max_seqlen_all, softmax_scale: Optional[float] = None, out_lo: Optional[Tensor] = None,
    split_flag: Optional[Tensor] = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Explicit backward: ``(dQ, dK, dV)`` from ``dO``, ``O`` and ``lse``.  For bf16, optionally the
    forward's low output half ``out_lo`` (delta = rowsum(dO * O) then exact to ~2^-17) and its
    recorded ``split_flag`` (the low half is then read only when the forward split)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else float(softmax_scale)
    lo = q.new_empty(0) if out_lo is None else out_lo
    flag = q.new_empty(0, dtype=torch.int32) if split_flag is None else split_flag
    return _prefixlm_bwd_op(dout, q, k, v, out, lse, lo, flag, bool(is_causal), prefix_lens, causal_lens,
                            cu_seqlens, _cpu_scalar(total_seqlen), _cpu_scalar(numseqs),
                            _cpu_scalar(max_seqlen_all), scale)


def flash_attn_varlen_prefixlm(
    q: Tensor,
    k: Tensor,
    v: Tensor,
    is_causal: bool,
    prefix_lens: Tensor,
    causal_lens: Tensor,
    cu_seqlens: Tensor,
    total_seqlen: Tensor,
    numseqs: Tensor,
    max_seqlen_prefix: Tensor,
    max_seqlen_causal: Tensor,
    max_seqlen_all: Tensor,
    *,
    prefix_cu_seqlens: Optional[Tensor] = None,
    prefix_idx: Optional[Tensor] = None,
    causal_idx: Optional[Tensor] = None,
    active_key_idx: Optional[Tensor] = None,
    active_cu_seqlens_q: Optional[Tensor] = None,
    active_cu_seqlens_k: Optional[Tensor] = None,
    cu_seqlens_shifted: Optional[Tensor] = None,
    prefix_mask: Optional[Tensor] = None,
    causal_mask: Optional[Tensor] = None,
    fa4_impl: str = "seqused",
    fa4_grad_mask_impl: str = "triton",
    fa4_output_combine_impl: str = "triton",
) -> Tensor:
    """Prefix-LM attention over packed sequences; returns O shaped like ``q``.

    Signature of src/mimir/model/flash_attention_prefixlm_v2.py:286-306.  One
    single-pass kernel covers both the bidirectional prefix block and the causal
    suffix, so the two-pass routing tensors (``prefix_idx`` ... ``causal_mask``)
    and the ``fa4_*`` knobs are accepted and ignored -- except that a partial set
    of the six routing tensors raises ``ValueError`` as the reference's gather
    backends do (flash_attention_prefixlm_rocm.py:71-72, fa4.py:505).
    ``max_seqlen_prefix`` / ``max_seqlen_causal`` are not needed by the kernels.
    """
    routing = (prefix_cu_seqlens, prefix_idx, causal_idx, active_key_idx, active_cu_seqlens_q, active_cu_seqlens_k)
    if any(r is None for r in routing) and not all(r is None for r in routing):
        raise ValueError(f"PrefixLM routing tensors must provide all of {ROUTING_KEYS}")
    out, _ = prefixlm_attn_fwd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                               max_seqlen_all)
    return out
