"""Packed prefix-LM batch metadata (host side).

Restates the metadata the reference builds for every packed batch so that a
caller of :func:`mimir_amd.flash_attn_varlen_prefixlm` can produce the same
arguments without the reference installed:

* :func:`compute_aux_seq_tensors_scalars` -- src/mimir/model/flash_attention_prefixlm_v2.py:21-35
  (tensors zero-padded to ``batch_max_tokens``; five python-int scalars).
* :class:`PrefixLMSeqInfo` / :func:`prefixlm_seq_info_from_tensors` --
  src/mimir/model/flash_attention_prefixlm_common.py:36-77 (slice padded
  metadata to ``numseqs``; ``cu_seqlens_shifted = cu_seqlens + pad(prefix_lens)``).
* :func:`prefixlm_prepared_from_tensors` -- src/mimir/model/flash_attention_prefixlm_common.py:87-133,
  the nine routing tensors that ``prepare_prefixlm_batch`` (src/mimir/model/common.py:36-70)
  adds to every batch for the ``sm100`` / ``rocm`` backends.  The kernels here
  take their tiles from ``cu_seqlens`` / ``prefix_lens`` and ignore them; they
  are restated so that a caller can pass the very keyword set Mimir2 passes.
* :func:`allowed_pairs` -- the per-sequence count of attended (query, key) pairs,
  ``(n^2 + n + p^2 - p) / 2``, used for the unmasked-FLOP accounting.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
from torch import Tensor

__all__ = [
    "PREFIXLM_ROUTING_KEYS",
    "PrefixLMSeqInfo",
    "allowed_pairs",
    "compute_aux_seq_tensors_scalars",
    "prefixlm_prepared_from_tensors",
    "prefixlm_seq_info_from_tensors",
]

# The keys prepare_prefixlm_batch adds (flash_attention_prefixlm_common.py:124-134).
PREFIXLM_ROUTING_KEYS = (
    "prefix_cu_seqlens",
    "prefix_idx",
    "causal_idx",
    "active_key_idx",
    "active_cu_seqlens_q",
    "active_cu_seqlens_k",
    "cu_seqlens_shifted",
    "prefix_mask",
    "causal_mask",
)


def compute_aux_seq_tensors_scalars(prefix_lens: np.ndarray, causal_lens: np.ndarray, batch_max_tokens: int):
    """Metadata for one packed row (flash_attention_prefixlm_v2.py:21-35).

    Returns ``(tensors, scalars)``: numpy arrays ``prefix_lens``, ``causal_lens``
    and ``cu_seqlens`` zero-padded to ``batch_max_tokens`` (``cu_seqlens`` has a
    leading 0), and python ints ``total_seqlen``, ``numseqs``,
    ``max_seqlen_prefix``, ``max_seqlen_causal``, ``max_seqlen_all``.
    """
    prefix_lens = np.asarray(prefix_lens)
    causal_lens = np.asarray(causal_lens)
    total_lens = prefix_lens + causal_lens
    n = total_lens.shape[0]
    tensors = {
        "prefix_lens": np.pad(prefix_lens, (0, batch_max_tokens - n)),
        "causal_lens": np.pad(causal_lens, (0, batch_max_tokens - n)),
        "cu_seqlens": np.pad(np.cumsum(total_lens, dtype=np.int32), (1, batch_max_tokens - n - 1)),
    }
    scalars = {
        "total_seqlen": int(total_lens.sum()),
        "numseqs": n,
        "max_seqlen_prefix": int(prefix_lens.max()),
        "max_seqlen_causal": int(causal_lens.max()),
        "max_seqlen_all": int(total_lens.max()),
    }
    return tensors, scalars


@dataclass(frozen=True)
class PrefixLMSeqInfo:
    total_seqlen: int
    numseqs: int
    max_seqlen_prefix: int
    max_seqlen_causal: int
    max_seqlen_all: int
    prefix_lens: Tensor
    causal_lens: Tensor
    cu_seqlens: Tensor
    cu_seqlens_shifted: Tensor


def _as_int(x) -> int:
    return int(x.item()) if isinstance(x, Tensor) else int(x)


def prefixlm_seq_info_from_tensors(
    prefix_lens: Tensor,
    causal_lens: Tensor,
    cu_seqlens: Tensor,
    total_seqlen,
    numseqs,
    max_seqlen_prefix,
    max_seqlen_causal,
    max_seqlen_all,
) -> PrefixLMSeqInfo:
    """Slice padded metadata to ``numseqs`` (flash_attention_prefixlm_common.py:49-77).

    The five scalars are CPU tensors (or ints) in the reference's convention, so
    reading them never synchronises the device.
    """
    nseq = _as_int(numseqs)
    cu = cu_seqlens[: nseq + 1]
    pl = prefix_lens[:nseq]
    cl = causal_lens[:nseq]
    shifted = cu + torch.nn.functional.pad(pl, (0, 1))
    return PrefixLMSeqInfo(
        total_seqlen=_as_int(total_seqlen),
        numseqs=nseq,
        max_seqlen_prefix=_as_int(max_seqlen_prefix),
        max_seqlen_causal=_as_int(max_seqlen_causal),
        max_seqlen_all=_as_int(max_seqlen_all),
        prefix_lens=pl,
        causal_lens=cl,
        cu_seqlens=cu,
        cu_seqlens_shifted=shifted,
    )


def prefixlm_prepared_from_tensors(prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs, max_seqlen_prefix,
                                   max_seqlen_causal, max_seqlen_all) -> dict:
    """The routing tensors of flash_attention_prefixlm_common.py:87-133 for one packed batch.

    Token t of sequence s at local position i is a prefix token when i < prefix_lens[s];
    ``prefix_idx`` / ``causal_idx`` list the prefix / causal tokens, ``active_key_idx``
    the tokens of sequences with a causal part, with their cumulative lengths.
    Built with device ops from device tensors (``repeat_interleave`` and boolean
    indexing synchronise once, as in the reference).
    """
    info = prefixlm_seq_info_from_tensors(prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                                          max_seqlen_prefix, max_seqlen_causal, max_seqlen_all)
    dev = info.prefix_lens.device
    prefix_cu = torch.nn.functional.pad(torch.cumsum(info.prefix_lens, dim=0, dtype=torch.int32), (1, 0))
    total_lens = info.prefix_lens + info.causal_lens
    seq_idx = torch.repeat_interleave(torch.arange(info.numseqs, device=dev), total_lens)
    valid_idx = torch.arange(info.total_seqlen, device=dev)
    token_idx = valid_idx - info.cu_seqlens[: info.numseqs][seq_idx]
    prefix_mask = token_idx < info.prefix_lens[seq_idx]
    active = info.causal_lens > 0
    causal_mask = (~prefix_mask) & active[seq_idx]
    return {
        "prefix_cu_seqlens": prefix_cu,
        "prefix_idx": valid_idx[prefix_mask],
        "causal_idx": valid_idx[causal_mask],
        "active_key_idx": valid_idx[active[seq_idx]],
        "active_cu_seqlens_q": torch.nn.functional.pad(
            torch.cumsum(info.causal_lens[active], dim=0, dtype=torch.int32), (1, 0)),
        "active_cu_seqlens_k": torch.nn.functional.pad(
            torch.cumsum(total_lens[active], dim=0, dtype=torch.int32), (1, 0)),
        "cu_seqlens_shifted": info.cu_seqlens_shifted,
        "prefix_mask": prefix_mask,
        "causal_mask": causal_mask,
    }


def allowed_pairs(seq_lens, prefix_lens, is_causal: bool = False) -> int:
    """Number of attended (query, key) pairs summed over sequences.

    For a sequence of length n with prefix p every query i sees kend(i) =
    max(p, i + 1) keys, so the count is sum_i max(p, i + 1) = (n^2 + n + p^2 - p) / 2
    (p = 0 for ``is_causal``).
    """
    n = np.asarray(seq_lens, dtype=np.int64)
    p = np.zeros_like(n) if is_causal else np.clip(np.asarray(prefix_lens, dtype=np.int64), 0, n)
    return int(((n * n + n + p * p - p) // 2).sum())
