"""Pins for the CPU oracle (no GPU).

The reference has no golden vectors for the attention operator, so each oracle
function is checked against statements it does not share code with: the
Metal predicate, the reference's own test stand-in mask, explicit fp64 loops,
closed forms, library special cases (SDPA causal / unmasked), autograd and
gradcheck, and invariants.  Each check is chosen so that a plausible slip
(mask off by one, wrong GQA head map, missing scale, wrong sign in dS, lse in
the wrong base) fails at least one of them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from mimir_amd.metadata import allowed_pairs
from mimir_amd.workloads import make_case
from oracle.prefixlm_oracle import (
    allowed,
    brute_force_backward,
    brute_force_forward,
    dense_backward,
    dense_forward,
    dense_forward_autograd,
    dense_lse,
    prefixlm_mask,
    repeat_kv,
)

F64 = torch.float64


def _case(seq_lens, prefixes, hq=4, hkv=2, d=8, seed=0, pad_to=None, is_causal=False, dtype=F64):
    return make_case(seq_lens, prefixes, hq, hkv, d, seed=seed, dtype=dtype, pad_to=pad_to, is_causal=is_causal)


# ---------------------------------------------------------------- mask
@pytest.mark.parametrize("n,p", [(1, 0), (1, 1), (5, 0), (5, 2), (5, 5), (9, 4), (16, 1), (16, 15)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_mask_matches_metal_predicate_and_stand_in(n, p, is_causal):
    m = prefixlm_mask(n, p, is_causal)
    # Metal predicate (flash_attention_prefixlm_mps.py:43-51), elementwise
    brute = torch.tensor([[allowed(is_causal, p, i, j) for j in range(n)] for i in range(n)])
    assert torch.equal(m, brute)
    # the reference test stand-in (tests/test_native_mimir2.py:27-30 with prefix 2, generalised to p)
    pos = torch.arange(n)
    pe = 0 if is_causal else p
    stand_in = (pos[:, None] >= pos[None, :]) | ((pos[:, None] < pe) & (pos[None, :] < pe))
    assert torch.equal(m, stand_in)
    # kend form used by the kernels: j < max(p, i + 1)
    kend = torch.clamp(pos + 1, min=pe)
    assert torch.equal(m, pos[None, :] < kend[:, None])
    assert int(m.sum()) == allowed_pairs([n], [p], is_causal)


def test_pair_count_closed_form():
    rng = np.random.default_rng(0)
    for _ in range(50):
        n = int(rng.integers(1, 300))
        p = int(rng.integers(0, n + 1))
        assert int(prefixlm_mask(n, p, False).sum()) == (n * n + n + p * p - p) // 2


# ---------------------------------------------------------------- forward
TINY = [
    ([5, 3, 1], [2, 3, 0], 4, 2, 8, None, False),
    ([6, 4], [0, 4], 2, 2, 4, 12, False),
    ([7], [3], 4, 1, 8, None, True),
    ([3, 0, 4], [1, 0, 2], 2, 1, 4, 9, False),
]


@pytest.mark.parametrize("idx", range(len(TINY)))
def test_forward_and_lse_match_brute_force(idx):
    seq, pre, hq, hkv, d, pad, causal = TINY[idx]
    c = _case(seq, pre, hq, hkv, d, seed=idx, pad_to=pad, is_causal=causal)
    o = dense_forward(c.q, c.k, c.v, causal, *c.oracle_args())
    lse = dense_lse(c.q, c.k, causal, *c.oracle_args())
    o_bf, lse_bf = brute_force_forward(c.q, c.k, c.v, causal, *c.oracle_args())
    np.testing.assert_allclose(o.numpy(), o_bf, atol=1e-12)
    np.testing.assert_allclose(lse.numpy(), lse_bf, atol=1e-12)


def test_chunked_forward_is_identical():
    c = _case([40, 25], [13, 25], 4, 2, 8, seed=4)
    a = dense_forward(c.q, c.k, c.v, False, *c.oracle_args())
    b = dense_forward(c.q, c.k, c.v, False, *c.oracle_args(), query_chunk=7)
    torch.testing.assert_close(a, b, atol=1e-12, rtol=0)


def _sdpa(q, k, v, **kw):
    return F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), **kw).transpose(0, 1)


def test_prefix_zero_is_causal_sdpa_and_full_prefix_is_unmasked():
    n = 23
    c0 = _case([n], [0], 2, 2, 8, seed=1)
    o = dense_forward(c0.q, c0.k, c0.v, False, *c0.oracle_args())
    torch.testing.assert_close(o, _sdpa(c0.q, c0.k, c0.v, is_causal=True), atol=1e-12, rtol=0)
    cn = _case([n], [n], 2, 2, 8, seed=1)
    o = dense_forward(cn.q, cn.k, cn.v, False, *cn.oracle_args())
    torch.testing.assert_close(o, _sdpa(cn.q, cn.k, cn.v), atol=1e-12, rtol=0)
    # is_causal ignores the prefix (flash_attention_prefixlm_dense.py:61-62)
    cp = _case([n], [9], 2, 2, 8, seed=1)
    o = dense_forward(cp.q, cp.k, cp.v, True, *cp.oracle_args())
    torch.testing.assert_close(o, _sdpa(cp.q, cp.k, cp.v, is_causal=True), atol=1e-12, rtol=0)


def test_gqa_head_map_is_repeat_interleave():
    c = _case([11], [4], 4, 2, 8, seed=2)
    o = dense_forward(c.q, c.k, c.v, False, *c.oracle_args())
    for h in range(4):
        g = h // 2  # q head h reads kv head h // (Hq / Hkv)
        oh = dense_forward(c.q[:, h:h + 1], c.k[:, g:g + 1], c.v[:, g:g + 1], False, *c.oracle_args())
        torch.testing.assert_close(o[:, h:h + 1], oh, atol=1e-12, rtol=0)
    k2, v2 = repeat_kv(c.q, c.k, c.v)
    assert torch.equal(k2[:, 1], c.k[:, 0]) and torch.equal(k2[:, 2], c.k[:, 1])


def test_softmax_rows_sum_to_one_and_padding_zero():
    c = _case([9, 5], [3, 0], 2, 1, 4, seed=3, pad_to=17)
    ones = torch.ones_like(c.v)
    o = dense_forward(c.q, c.k, ones, False, *c.oracle_args())
    torch.testing.assert_close(o[:14], torch.ones_like(o[:14]), atol=1e-12, rtol=0)
    assert torch.count_nonzero(o[14:]) == 0
    lse = dense_lse(c.q, c.k, False, *c.oracle_args())
    assert torch.isneginf(lse[:, 14:]).all()


def test_documents_are_independent():
    c = _case([8, 6, 7], [2, 6, 0], 2, 2, 4, seed=5)
    o = dense_forward(c.q, c.k, c.v, False, *c.oracle_args())
    q2, k2, v2 = c.q.clone(), c.k.clone(), c.v.clone()
    q2[8:14] += 3.0
    k2[8:14] -= 1.0
    v2[8:14] *= 2.0
    o2 = dense_forward(q2, k2, v2, False, *c.oracle_args())
    torch.testing.assert_close(o[:8], o2[:8], atol=0, rtol=0)
    torch.testing.assert_close(o[14:], o2[14:], atol=0, rtol=0)
    assert not torch.allclose(o[8:14], o2[8:14])


def test_prefix_permutation_equivariance():
    n, p = 12, 7
    c = _case([n], [p], 2, 2, 8, seed=6)
    o = dense_forward(c.q, c.k, c.v, False, *c.oracle_args())
    perm = torch.cat([torch.randperm(p, generator=torch.Generator().manual_seed(0)), torch.arange(p, n)])
    o2 = dense_forward(c.q[perm], c.k[perm], c.v[perm], False, *c.oracle_args())
    torch.testing.assert_close(o2, o[perm], atol=1e-12, rtol=0)


def test_lse_single_key_closed_form():
    c = _case([6], [0], 2, 2, 8, seed=7)
    lse = dense_lse(c.q, c.k, False, *c.oracle_args())
    # query 0 with p = 0 sees only key 0: lse = scale * q0 . k0 (natural log)
    expect = (c.q[0] * c.k[0]).sum(-1) / math.sqrt(8)
    torch.testing.assert_close(lse[:, 0], expect, atol=1e-12, rtol=0)


def test_bad_lengths_raise_value_error():
    c = _case([5, 3], [2, 3], 2, 2, 4)
    bad = c.causal_lens.clone()
    bad[0] += 1
    with pytest.raises(ValueError, match="Bad PrefixLM lengths"):
        dense_forward(c.q, c.k, c.v, False, c.prefix_lens, bad, c.cu_seqlens, c.total_seqlen, c.numseqs)


# ---------------------------------------------------------------- backward
@pytest.mark.parametrize("idx", range(len(TINY)))
def test_backward_matches_autograd_and_brute_force(idx):
    seq, pre, hq, hkv, d, pad, causal = TINY[idx]
    c = _case(seq, pre, hq, hkv, d, seed=10 + idx, pad_to=pad, is_causal=causal)
    q, k, v = (t.clone().requires_grad_(True) for t in (c.q, c.k, c.v))
    o = dense_forward_autograd(q, k, v, causal, *c.oracle_args())
    o.backward(c.dout)
    dq, dk, dv = dense_backward(c.q, c.k, c.v, o.detach(), c.dout, causal, *c.oracle_args())
    torch.testing.assert_close(dq, q.grad, atol=1e-11, rtol=0)
    torch.testing.assert_close(dk, k.grad, atol=1e-11, rtol=0)
    torch.testing.assert_close(dv, v.grad, atol=1e-11, rtol=0)
    bq, bk, bv = brute_force_backward(c.q, c.k, c.v, c.dout, causal, *c.oracle_args())
    np.testing.assert_allclose(dq.numpy(), bq, atol=1e-11)
    np.testing.assert_allclose(dk.numpy(), bk, atol=1e-11)
    np.testing.assert_allclose(dv.numpy(), bv, atol=1e-11)


def test_gradcheck_fp64():
    c = _case([4, 3], [2, 1], 2, 1, 4, seed=20, pad_to=8)
    q, k, v = (t.clone().requires_grad_(True) for t in (c.q, c.k, c.v))
    fn = lambda q_, k_, v_: dense_forward_autograd(q_, k_, v_, False, *c.oracle_args())
    assert torch.autograd.gradcheck(fn, (q, k, v), eps=1e-6, atol=1e-7)


def test_padding_rows_get_no_query_gradient():
    c = _case([6, 4], [3, 0], 2, 2, 4, seed=21, pad_to=13)
    dq, dk, dv = dense_backward(c.q, c.k, c.v, dense_forward(c.q, c.k, c.v, False, *c.oracle_args()), c.dout,
                                False, *c.oracle_args())
    assert torch.count_nonzero(dq[10:]) == 0
    assert torch.count_nonzero(dk[10:]) == 0 and torch.count_nonzero(dv[10:]) == 0


# ---------------------------------------------------------------- chunked closed form
def _with_total(case, total):
    case.total_seqlen = torch.tensor(int(total), dtype=torch.int64)
    return case


@pytest.mark.parametrize("chunk", [1, 3, 7, 64])
@pytest.mark.parametrize("shape", [
    # seq_lens, prefixes, hq, hkv, pad_to, is_causal, total (None: all tokens)
    ([9, 1, 12], [4, 1, 0], 4, 2, 25, False, None),
    ([9, 1, 12], [4, 1, 0], 4, 4, None, True, None),
    ([16, 7], [16, 3], 6, 2, None, False, 20),     # total ends inside the second sequence, past its prefix
    ([16, 7], [5, 3], 2, 1, None, False, 3),       # total ends inside the first sequence's prefix
])
def test_chunked_forward_backward_equals_dense(chunk, shape):
    """The chunked restatement equals the per-sequence dense forward, the closed-form lse and
    the closed-form backward (all fp64), for every chunk size: a dropped mask term, a wrong
    chunk boundary, a missing GQA sum or a wrong delta would show."""
    from oracle.prefixlm_oracle import chunked_forward_backward

    seq_lens, prefixes, hq, hkv, pad_to, causal, total = shape
    c = _case(seq_lens, prefixes, hq=hq, hkv=hkv, d=8, seed=7, pad_to=pad_to, is_causal=causal)
    if total is not None:
        _with_total(c, total)
    args = c.oracle_args()
    o_ref = dense_forward(c.q, c.k, c.v, causal, *args)
    lse_ref = dense_lse(c.q, c.k, causal, *args)
    dq_ref, dk_ref, dv_ref = dense_backward(c.q, c.k, c.v, o_ref, c.dout, causal, *args)
    o, lse, dq, dk, dv = chunked_forward_backward(c.q, c.k, c.v, c.dout, causal, *args, chunk=chunk)
    for got, ref in ((o, o_ref), (dq, dq_ref), (dk, dk_ref), (dv, dv_ref)):
        torch.testing.assert_close(got, ref, rtol=1e-12, atol=1e-12)
    fin = torch.isfinite(lse_ref)
    assert torch.equal(fin, torch.isfinite(lse))
    torch.testing.assert_close(lse[fin], lse_ref[fin], rtol=1e-12, atol=1e-12)


def test_backward_with_total_inside_a_sequence_matches_autograd():
    """total_seqlen ending inside a sequence past its prefix: O rows from total on are zero
    (dense.py:79-80), so no gradient flows from them, while the keys there stay keys for
    earlier prefix rows.  The closed form agrees with autograd through dense_forward."""
    c = _with_total(_case([12, 9], [8, 2], hq=4, hkv=2, d=8, seed=3), 16)
    args = c.oracle_args()
    q, k, v = (t.clone().requires_grad_(True) for t in (c.q, c.k, c.v))
    dense_forward_autograd(q, k, v, False, *args).backward(c.dout)
    o = dense_forward(c.q, c.k, c.v, False, *args)
    dq, dk, dv = dense_backward(c.q, c.k, c.v, o, c.dout, False, *args)
    for got, ref in ((dq, q.grad), (dk, k.grad), (dv, v.grad)):
        torch.testing.assert_close(got, ref, rtol=1e-10, atol=1e-10)
    # keys of the second sequence past total still receive gradient from its prefix rows
    assert dk[12 + 4:12 + 8].abs().sum() == 0  # keys 4..7 of seq 2 are in its causal part: rows >= 4 only
    assert dq[16:].abs().sum() == 0
