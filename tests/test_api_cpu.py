"""Host-side API checks (no GPU): metadata helpers, argument handling of the
drop-in entry point, and the seeded workload generator."""

import numpy as np
import pytest
import torch

import mimir_amd
from mimir_amd import (
    allowed_pairs,
    compute_aux_seq_tensors_scalars,
    flash_attn_varlen_prefixlm,
    prefixlm_seq_info_from_tensors,
)
from mimir_amd.workloads import bwd_bytes, fwd_bytes, make_case, make_config
from oracle.prefixlm_oracle import prefixlm_mask


def test_metadata_matches_reference_example():
    # the call made by tests/test_v2_extensions.py:266-267 of the reference
    tensors, scalars = compute_aux_seq_tensors_scalars(np.array([1, 2], dtype=np.int32),
                                                       np.array([2, 3], dtype=np.int32), 8)
    np.testing.assert_array_equal(tensors["prefix_lens"], [1, 2, 0, 0, 0, 0, 0, 0])
    np.testing.assert_array_equal(tensors["causal_lens"], [2, 3, 0, 0, 0, 0, 0, 0])
    np.testing.assert_array_equal(tensors["cu_seqlens"], [0, 3, 8, 0, 0, 0, 0, 0])
    assert tensors["cu_seqlens"].dtype == np.int32
    assert scalars == {"total_seqlen": 8, "numseqs": 2, "max_seqlen_prefix": 2, "max_seqlen_causal": 3,
                       "max_seqlen_all": 5}


def test_seq_info_slices_and_shifts():
    tensors, scalars = compute_aux_seq_tensors_scalars(np.array([3, 0, 5]), np.array([4, 2, 1]), 16)
    t = {k: torch.from_numpy(v) for k, v in tensors.items()}
    s = {k: torch.tensor(v) for k, v in scalars.items()}
    info = prefixlm_seq_info_from_tensors(**t, **s)
    assert info.numseqs == 3 and info.total_seqlen == 15
    assert info.cu_seqlens.tolist() == [0, 7, 9, 15]
    assert info.prefix_lens.tolist() == [3, 0, 5]
    assert info.cu_seqlens_shifted.tolist() == [3, 7, 14, 15]


@pytest.mark.parametrize("causal", [False, True])
def test_allowed_pairs_counts_mask(causal):
    rng = np.random.default_rng(1)
    n = rng.integers(1, 200, size=6)
    p = np.array([rng.integers(0, x + 1) for x in n])
    brute = sum(int(prefixlm_mask(int(a), int(b), causal).sum()) for a, b in zip(n, p))
    assert allowed_pairs(n, p, causal) == brute


def test_cpu_tensors_raise_no_fallback():
    c = make_case([8], [3], 2, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPUs only"):
        flash_attn_varlen_prefixlm(c.q, c.k, c.v, False, *c.call_args())


def test_partial_routing_tensors_raise():
    c = make_case([8], [3], 2, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="routing tensors"):
        flash_attn_varlen_prefixlm(c.q, c.k, c.v, False, *c.call_args(), prefix_idx=torch.arange(3))


def test_signature_matches_reference_keywords():
    import inspect

    params = inspect.signature(flash_attn_varlen_prefixlm).parameters
    positional = ["q", "k", "v", "is_causal", "prefix_lens", "causal_lens", "cu_seqlens", "total_seqlen", "numseqs",
                  "max_seqlen_prefix", "max_seqlen_causal", "max_seqlen_all"]
    keywords = ["prefix_cu_seqlens", "prefix_idx", "causal_idx", "active_key_idx", "active_cu_seqlens_q",
                "active_cu_seqlens_k", "cu_seqlens_shifted", "prefix_mask", "causal_mask", "fa4_impl",
                "fa4_grad_mask_impl", "fa4_output_combine_impl"]
    assert list(params)[:12] == positional
    assert list(params)[12:] == keywords
    assert all(params[k].kind is inspect.Parameter.KEYWORD_ONLY for k in keywords)


def test_custom_ops_registered_with_fake_kernels():
    assert hasattr(torch.ops.mimir_amd, "prefixlm_fwd") and hasattr(torch.ops.mimir_amd, "prefixlm_bwd")
    c = make_case([6, 10], [2, 10], 4, 2, 64, dtype=torch.bfloat16)
    meta = (c.prefix_lens, c.causal_lens, c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, 0.125)
    with torch._subclasses.fake_tensor.FakeTensorMode(allow_non_fake_inputs=True):
        q = torch.empty(16, 4, 64, dtype=torch.bfloat16)
        k = torch.empty(16, 2, 64, dtype=torch.bfloat16)
        out, lse, lo, flag = torch.ops.mimir_amd.prefixlm_fwd(q, k, k, False, *meta)
        assert out.shape == (16, 4, 64) and lse.shape == (4, 16) and lse.dtype == torch.float32
        assert lo.shape == out.shape and lo.dtype == torch.bfloat16
        assert flag.shape == (1,) and flag.dtype == torch.int32
        dq, dk, dv = torch.ops.mimir_amd.prefixlm_bwd(out, q, k, k, out, lse, lo, flag, False, *meta)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape and dk.dtype == torch.bfloat16
        qf = torch.empty(16, 4, 64)
        kf = torch.empty(16, 2, 64)
        out, lse, lo, flag = torch.ops.mimir_amd.prefixlm_fwd(qf, kf, kf, False, *meta)
        assert lo.numel() == 0 and flag.numel() == 0  # float32 carries no low half and no split


def test_forward_and_backward_trace_with_fake_tensors():
    """The drop-in with autograd traced by make_fx in fake mode: forward and backward become
    exactly one call each of the two custom ops, shaped by their fake kernels alone (no device
    work, no data-dependent host reads), as torch.compile would see them."""
    from torch.fx.experimental.proxy_tensor import make_fx

    c = make_case([6, 10], [2, 10], 4, 2, 64, dtype=torch.bfloat16)

    def step(q, k, v, dout, *meta):
        out = flash_attn_varlen_prefixlm(q, k, v, False, *meta)
        return torch.autograd.grad(out, (q, k, v), dout)

    args = (torch.randn(16, 4, 64, dtype=torch.bfloat16, requires_grad=True),
            torch.randn(16, 2, 64, dtype=torch.bfloat16, requires_grad=True),
            torch.randn(16, 2, 64, dtype=torch.bfloat16, requires_grad=True),
            torch.randn(16, 4, 64, dtype=torch.bfloat16)) + c.call_args()
    gm = make_fx(step, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert sum("mimir_amd.prefixlm_fwd" in t for t in targets) == 1, targets
    assert sum("mimir_amd.prefixlm_bwd" in t for t in targets) == 1, targets


@pytest.mark.parametrize("idx", [1, 2, 3])
def test_workload_generator(idx):
    c = make_config(idx, seed=0)
    T = c.q.shape[0]
    n, p = np.array(c.seq_lens), np.array(c.prefixes)
    assert n.sum() == int(c.total_seqlen) <= T
    assert ((p >= 0) & (p <= n)).all()
    assert (c.prefix_lens[: len(n)].numpy() + c.causal_lens[: len(n)].numpy() == n).all()
    assert c.cu_seqlens[len(n)].item() == n.sum()
    if idx == 3:
        assert T == 16384 and n.sum() == 16384 and (n[:-1] >= 128).all() and (n <= 4096).all()
    again = make_config(idx, seed=0)
    assert torch.equal(c.q, again.q) and c.prefixes == again.prefixes


def test_work_accounting_matches_baseline_table():
    # config 2 bytes: fwd 168.8 MB + bwd 338.7 MB (bf16, T=16384, Hq=16, Hkv=4, D=128)
    assert abs(fwd_bytes(16384, 16, 4, 128, 2) / 1e6 - 168.8) < 0.1
    assert abs(bwd_bytes(16384, 16, 4, 128, 2) / 1e6 - 338.7) < 0.1
    # config 4 pairs: n = 32768, p = 8192
    assert allowed_pairs([32768], [8192]) == 570437632


def test_package_exports():
    for name in mimir_amd.__all__:
        assert hasattr(mimir_amd, name)


def test_cache_attention_argument_checks_on_cpu():
    """attention_with_cache (layers.py:134-167) checks dtype and shapes before anything runs, and CPU
    tensors raise instead of falling back."""
    from mimir_amd.cache import Cache, attention_with_cache
    bf = torch.bfloat16
    q = torch.zeros(2, 1, 8, 64, dtype=bf)
    k = torch.zeros(2, 1, 2, 64, dtype=bf)
    cache = Cache.create(2, 16, 2, 64, dtype=bf)
    assert cache.keys.shape == (2, 16, 2, 64) and cache.values.dtype == bf and not cache.keys.any()
    lens = torch.tensor([3, 0])
    with pytest.raises(TypeError):
        attention_with_cache(q.float(), k.float(), k.float(), Cache.create(2, 16, 2, 64), lens, True)
    with pytest.raises(ValueError):  # key / value shapes differ from the query's batch and tokens
        attention_with_cache(q, k[:1], k[:1], cache, lens, True)
    with pytest.raises(ValueError):  # Hq not a multiple of Hkv
        attention_with_cache(torch.zeros(2, 1, 3, 64, dtype=bf), k, k, cache, lens, True)
    with pytest.raises(ValueError):  # cache head_dim differs
        attention_with_cache(q, k, k, Cache.create(2, 16, 2, 32, dtype=bf), lens, True)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        attention_with_cache(q, k, k, cache, lens, True)


def test_layer_core_cpu_tensors_raise():
    """The fused layer core (layers.py:182-239) and the RoPE kernel have no CPU fallback either."""
    from mimir_amd import rope
    x = torch.zeros(4, 2, 64, dtype=torch.bfloat16)
    cs = torch.ones(4, 64)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        rope(x, cs, cs)
