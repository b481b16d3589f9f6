"""CPU oracle for Mimir2 prefix-LM attention.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as what
the kernels' results are compared against (or, for the baseline, as the timed
CPU restatement of the reference's masked-SDPA path).  The product path (``mimir_amd``) never imports it: it runs
the HIP library or raises.

Every function restates the reference algorithm it cites.  The reference is
pure Python/torch; its operator path has no golden vectors or known-answer
tests (no test imports the attention backends), so each function here is pinned
by independent checks in ``tests/test_oracle.py``:

=============================  ===================================================
function                        pinned by
=============================  ===================================================
``prefixlm_mask``               the Metal predicate restated elementwise
                                (``allowed``), the reference test stand-in with a
                                2-token prefix, closed-form pair count
``dense_forward``               fp64 brute-force loops (``brute_force_forward``),
                                p = 0 == SDPA(is_causal=True), p = n == unmasked
                                SDPA, GQA == repeated KV, softmax rows sum to 1,
                                document independence, prefix permutation
``dense_lse``                   brute force; logsumexp of a single allowed key
``dense_backward``              torch.autograd of ``dense_forward`` in fp64,
                                ``torch.autograd.gradcheck``, brute-force loops
``chunked_forward_backward``    equality with ``dense_forward`` / ``dense_lse`` /
                                ``dense_backward`` (chunked == unchunked, every
                                chunk size, GQA, padding rows, is_causal)
=============================  ===================================================

``chunked_forward_backward`` evaluates the same closed forms query-chunk by
query-chunk and head by head, so a 32k-token sequence never needs more than a
chunk x n score matrix; it takes any floating dtype and device (the long-context
parity test runs it in float64 on the GPU through torch's own matmul, not
through anything of the product).
"""

from __future__ import annotations

import math
import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

__all__ = [
    "allowed",
    "brute_force_backward",
    "brute_force_forward",
    "chunked_forward_backward",
    "dense_backward",
    "dense_forward",
    "dense_forward_autograd",
    "dense_lse",
    "prefixlm_mask",
    "repeat_kv",
]


# ---------------------------------------------------------------------------
# Mask
# ---------------------------------------------------------------------------
def allowed(is_causal: bool, prefix_len: int, query_pos: int, key_pos: int) -> bool:
    """Scalar predicate, flash_attention_prefixlm_mps.py:43-51."""
    if is_causal:
        return key_pos <= query_pos
    if query_pos < prefix_len:
        return key_pos < prefix_len
    return key_pos <= query_pos


def prefixlm_mask(seq_len: int, prefix_len: int, is_causal: bool, device=None) -> Tensor:
    """Boolean [n, n] mask, True = attend (flash_attention_prefixlm_dense.py:59-69)."""
    positions = torch.arange(seq_len, device=device)
    if is_causal:
        return positions[None, :] <= positions[:, None]
    prefix_queries = positions < prefix_len
    prefix_keys = positions < prefix_len
    causal_queries = ~prefix_queries
    return (prefix_queries[:, None] & prefix_keys[None, :]) | (
        causal_queries[:, None] & (positions[None, :] <= positions[:, None])
    )


def repeat_kv(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor]:
    """GQA by repeat_interleave over heads (flash_attention_prefixlm_dense.py:10-16)."""
    if q.shape[-2] == k.shape[-2]:
        return k, v
    if q.shape[-2] % k.shape[-2] != 0:
        raise ValueError(f"Query heads {q.shape[-2]} must be divisible by key/value heads {k.shape[-2]}.")
    rep = q.shape[-2] // k.shape[-2]
    return k.repeat_interleave(rep, dim=-2), v.repeat_interleave(rep, dim=-2)


def _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
    """(start, end, prefix) per sequence; slicing of flash_attention_prefixlm_common.py:59-65."""
    n = int(numseqs)
    cu = [int(x) for x in cu_seqlens[: n + 1].tolist()]
    pl = [int(x) for x in prefix_lens[:n].tolist()]
    cl = [int(x) for x in causal_lens[:n].tolist()]
    out = []
    for s in range(n):
        start, end = cu[s], cu[s + 1]
        if end - start == 0:
            continue
        if pl[s] + cl[s] != end - start:
            raise ValueError(f"Bad PrefixLM lengths for sequence {s}: {pl[s]} + {cl[s]} != {end - start}")
        out.append((start, end, pl[s]))
    return out


# ---------------------------------------------------------------------------
# Forward (masked SDPA per sequence) -- flash_attention_prefixlm_dense.py:19-81
# ---------------------------------------------------------------------------
def dense_forward(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                  query_chunk: int | None = None) -> Tensor:
    """Output O of the reference's dense path, in the dtype of ``q``.

    ``query_chunk`` splits each sequence's queries into blocks of that many rows
    (identical math: every query row's softmax is independent) so long sequences
    never materialise an n x n score matrix.
    """
    out = torch.zeros_like(q)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        n = end - start
        q_seq = q[start:end]
        k_seq, v_seq = repeat_kv(q_seq, k[start:end], v[start:end])
        mask = prefixlm_mask(n, p, is_causal, device=q.device)
        kt = k_seq.transpose(0, 1).unsqueeze(0)
        vt = v_seq.transpose(0, 1).unsqueeze(0)
        step = n if query_chunk is None else query_chunk
        for a in range(0, n, step):
            b = min(n, a + step)
            kend = b if is_causal else max(p, b)  # keys beyond kend are masked for every row of the block
            attn = F.scaled_dot_product_attention(
                q_seq[a:b].transpose(0, 1).unsqueeze(0),
                kt[:, :, :kend],
                vt[:, :, :kend],
                attn_mask=mask[a:b, :kend].unsqueeze(0).unsqueeze(0),
            )
            out[start + a:start + b] = attn.squeeze(0).transpose(0, 1)
    total = int(total_seqlen)
    if total < q.shape[0]:
        out[total:] = 0
    return out


def dense_forward_autograd(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs):
    """Differentiable :func:`dense_forward`: slice assignment into a zero buffer,
    as the reference does (flash_attention_prefixlm_dense.py:43,77,79-80)."""
    out = torch.zeros_like(q)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        n = end - start
        q_seq = q[start:end]
        k_seq, v_seq = repeat_kv(q_seq, k[start:end], v[start:end])
        mask = prefixlm_mask(n, p, is_causal, device=q.device)
        attn = F.scaled_dot_product_attention(
            q_seq.transpose(0, 1).unsqueeze(0),
            k_seq.transpose(0, 1).unsqueeze(0),
            v_seq.transpose(0, 1).unsqueeze(0),
            attn_mask=mask.unsqueeze(0).unsqueeze(0),
        )
        out[start:end] = attn.squeeze(0).transpose(0, 1)
    total = int(total_seqlen)
    if total < q.shape[0]:
        out[total:] = 0
    return out


def dense_lse(q, k, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
              scale: float | None = None) -> Tensor:
    """Closed-form logsumexp [Hq, T]: ln sum_{j allowed} exp(scale * q_i . k_j).

    Rows outside every sequence or at/after ``total_seqlen`` are -inf (empty sum).
    The Metal kernels define the same quantity as m + log(l)
    (flash_attention_prefixlm_mps.py:385-388, 473-475).
    """
    T, hq, d = q.shape
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    lse = torch.full((hq, T), float("-inf"), dtype=q.dtype, device=q.device)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        n = end - start
        k_seq, _ = repeat_kv(q[start:end], k[start:end], k[start:end])
        scores = torch.einsum("ihd,jhd->hij", q[start:end], k_seq) * scale
        mask = prefixlm_mask(n, p, is_causal, device=q.device)
        scores = scores.masked_fill(~mask.unsqueeze(0), float("-inf"))
        lse[:, start:end] = torch.logsumexp(scores, dim=-1)
    total = int(total_seqlen)
    if total < T:
        lse[:, total:] = float("-inf")
    return lse


# ---------------------------------------------------------------------------
# Backward -- closed form of flash_attention_prefixlm_mps.py:1601-1675, with the
# GQA reduction (sum over the q heads of each kv head) that repeat_interleave's
# backward implies (flash_attention_prefixlm_dense.py:10-16).
# ---------------------------------------------------------------------------
def dense_backward(q, k, v, out, dout, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs,
                   scale: float | None = None):
    T, hq, d = q.shape
    hkv = k.shape[1]
    rep = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    total = int(total_seqlen)
    dout = dout.clone()
    if total < T:
        dout[total:] = 0  # O rows >= total_seqlen are overwritten with 0: no gradient flows (dense.py:79-80)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        n = end - start
        qs = q[start:end].transpose(0, 1)                       # [Hq, n, d]
        ks = k[start:end].repeat_interleave(rep, dim=1).transpose(0, 1)
        vs = v[start:end].repeat_interleave(rep, dim=1).transpose(0, 1)
        os_ = out[start:end].transpose(0, 1)
        dos = dout[start:end].transpose(0, 1)
        scores = torch.matmul(qs, ks.transpose(-1, -2)) * scale
        mask = prefixlm_mask(n, p, is_causal, device=q.device)
        scores = scores.masked_fill(~mask.unsqueeze(0), float("-inf"))
        prob = torch.softmax(scores, dim=-1)
        dv_rep = torch.matmul(prob.transpose(-1, -2), dos)
        dprob = torch.matmul(dos, vs.transpose(-1, -2))
        delta = (dos * os_).sum(dim=-1, keepdim=True)
        dscores = prob * (dprob - delta) * scale
        dq_s = torch.matmul(dscores, ks)
        dk_rep = torch.matmul(dscores.transpose(-1, -2), qs)
        dq[start:end] = dq_s.transpose(0, 1)
        dk[start:end] = dk_rep.reshape(hkv, rep, n, d).sum(1).transpose(0, 1)
        dv[start:end] = dv_rep.reshape(hkv, rep, n, d).sum(1).transpose(0, 1)
    return dq, dk, dv


def chunked_forward_backward(q, k, v, dout, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen,
                             numseqs, scale: float | None = None, chunk: int = 4096):
    """O, lse, dQ, dK, dV of the reference's masked attention from (q, k, v, dO) alone.

    The closed forms of :func:`dense_forward`, :func:`dense_lse` and
    :func:`dense_backward` (flash_attention_prefixlm_dense.py:19-81 and the
    backward of flash_attention_prefixlm_mps.py:1601-1675 with the GQA sum of
    dense.py:10-16), evaluated per sequence, q head and block of ``chunk`` query
    rows: S = scale Q K^T over the keys the block can see, P = exp(S - lse),
    O = P V, delta = rowsum(dO * O) from this O, dS = P (dO V^T - delta) * scale,
    dQ = dS K, dK += dS^T Q, dV += P^T dO.  Rows at or after ``total_seqlen`` get
    O = 0, lse = -inf and no gradient (dense.py:79-80).  Works in the dtype and on
    the device of the inputs.
    """
    T, hq, d = q.shape
    hkv = k.shape[1]
    rep = hq // hkv
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    total = int(total_seqlen)
    out = torch.zeros_like(q)
    lse = torch.full((hq, T), float("-inf"), dtype=q.dtype, device=q.device)
    dq = torch.zeros_like(q)
    dk = torch.zeros_like(k)
    dv = torch.zeros_like(v)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        n = end - start
        nq = max(0, min(n, total - start))
        pos = torch.arange(n, device=q.device)
        for h in range(hq):
            g = h // rep
            ks, vs = k[start:end, g], v[start:end, g]                      # [n, d]
            for a in range(0, nq, chunk):
                b = min(nq, a + chunk)
                kend = b if is_causal else max(p, b)                        # keys any row of the block sees
                qs, dos = q[start + a:start + b, h], dout[start + a:start + b, h]
                kc, vc = ks[:kend], vs[:kend]
                sc = torch.matmul(qs, kc.transpose(0, 1).contiguous()) * scale
                rows = pos[a:b, None]
                cols = pos[None, :kend]
                allowed = cols <= rows if is_causal else (cols < torch.clamp(rows + 1, min=p))
                sc = sc.masked_fill(~allowed, float("-inf"))
                l_ = torch.logsumexp(sc, dim=1)
                pr = torch.exp(sc - l_[:, None])
                o = torch.matmul(pr, vc)
                delta = (dos * o).sum(dim=1, keepdim=True)
                ds = pr * (torch.matmul(dos, vc.transpose(0, 1).contiguous()) - delta) * scale
                out[start + a:start + b, h] = o
                lse[h, start + a:start + b] = l_
                dq[start + a:start + b, h] = torch.matmul(ds, kc)
                dk[start:start + kend, g] += torch.matmul(ds.transpose(0, 1).contiguous(), qs)
                dv[start:start + kend, g] += torch.matmul(pr.transpose(0, 1).contiguous(), dos)
    return out, lse, dq, dk, dv


# ---------------------------------------------------------------------------
# Brute force (pure Python loops, fp64): for tiny shapes only.
# ---------------------------------------------------------------------------
def _np(x):
    return np.asarray(x.detach().cpu().double().numpy() if isinstance(x, Tensor) else x, dtype=np.float64)


def brute_force_forward(q, k, v, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs):
    """O and lse by explicit loops over (query, head, key) with the scalar predicate."""
    qn, kn, vn = _np(q), _np(k), _np(v)
    T, hq, d = qn.shape
    hkv = kn.shape[1]
    scale = 1.0 / math.sqrt(d)
    o = np.zeros_like(qn)
    lse = np.full((hq, T), -np.inf)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        for i in range(end - start):
            if start + i >= int(total_seqlen):
                continue
            for h in range(hq):
                g = h // (hq // hkv)
                js = [j for j in range(end - start) if allowed(is_causal, p, i, j)]
                s = [scale * sum(qn[start + i, h, x] * kn[start + j, g, x] for x in range(d)) for j in js]
                m = max(s)
                w = [math.exp(t - m) for t in s]
                z = sum(w)
                for x in range(d):
                    o[start + i, h, x] = sum(wj * vn[start + j, g, x] for wj, j in zip(w, js)) / z
                lse[h, start + i] = m + math.log(z)
    return o, lse


def brute_force_backward(q, k, v, dout, is_causal, prefix_lens, causal_lens, cu_seqlens, total_seqlen, numseqs):
    """dQ, dK, dV by explicit loops: dS_ij = P_ij (dO_i . V_j - sum_j' P_ij' dO_i . V_j')."""
    qn, kn, vn, don = _np(q), _np(k), _np(v), _np(dout)
    T, hq, d = qn.shape
    hkv = kn.shape[1]
    scale = 1.0 / math.sqrt(d)
    dq, dk, dv = np.zeros_like(qn), np.zeros_like(kn), np.zeros_like(vn)
    for start, end, p in _seqs(prefix_lens, causal_lens, cu_seqlens, numseqs):
        for i in range(end - start):
            if start + i >= int(total_seqlen):
                continue
            for h in range(hq):
                g = h // (hq // hkv)
                js = [j for j in range(end - start) if allowed(is_causal, p, i, j)]
                s = [scale * float(np.dot(qn[start + i, h], kn[start + j, g])) for j in js]
                m = max(s)
                w = [math.exp(t - m) for t in s]
                z = sum(w)
                pr = [x / z for x in w]
                dp = [float(np.dot(don[start + i, h], vn[start + j, g])) for j in js]
                mean = sum(a * b for a, b in zip(pr, dp))
                for pj, dpj, j in zip(pr, dp, js):
                    ds = pj * (dpj - mean) * scale
                    dq[start + i, h] += ds * kn[start + j, g]
                    dk[start + j, g] += ds * qn[start + i, h]
                    dv[start + j, g] += pj * don[start + i, h]
    return dq, dk, dv
