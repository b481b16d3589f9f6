"""GPU parity of the KV-cache attention (mimir_amd.cache, inference path of
src/mimir/model/layers.py:134-167) against the oracle's restatement.

Tolerances: output <= 2e-2 max-abs (the bf16 operator bar; the oracle runs in
fp32 on the same bf16 values); the cache writes are exact copies and every other
cache position is left untouched.  Cases cover decode (S = 1, key range split
over workgroups and merged), chunked prefill into a non-empty cache (causal and
bidirectional), GQA, batch_indices, an unsplit launch, and the IndexError of a
write past the cache.
"""

import pytest
import torch

from mimir_amd.cache import Cache, attention_with_cache
from oracle import layer_oracle as LO

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _run(device, B, S, hq, hkv, d, L, lens, causal, rows=None, cache_rows=None, seed=0, index_dtype=torch.int64):
    gen = torch.Generator().manual_seed(seed)
    cache_rows = cache_rows or B
    q = torch.randn(B, S, hq, d, generator=gen).to(BF16)
    k = torch.randn(B, S, hkv, d, generator=gen).to(BF16)
    v = torch.randn(B, S, hkv, d, generator=gen).to(BF16)
    ck = torch.randn(cache_rows, L, hkv, d, generator=gen).to(BF16)
    cv = torch.randn(cache_rows, L, hkv, d, generator=gen).to(BF16)
    lens_t = torch.tensor(lens, dtype=index_dtype)
    rows_t = None if rows is None else torch.tensor(rows, dtype=index_dtype)
    ck_ref, cv_ref = ck.clone(), cv.clone()
    ref = LO.attention_with_cache(q, k, v, ck_ref, cv_ref, lens_t, causal, rows_t)

    cache = Cache(ck.to(device), cv.to(device))
    out = attention_with_cache(q.to(device), k.to(device), v.to(device), cache, lens_t.to(device), causal,
                               None if rows_t is None else rows_t.to(device))
    torch.cuda.synchronize()
    err = (out.float().cpu() - ref.float()).abs().max().item()
    print(f"[cache] B={B} S={S} hq={hq} hkv={hkv} d={d} L={L} lens={lens} causal={causal} err={err:.3g}", flush=True)
    assert err <= 2e-2
    assert torch.equal(cache.keys.cpu(), ck_ref) and torch.equal(cache.values.cpu(), cv_ref)


@pytest.mark.parametrize("d", [128, 64])
@pytest.mark.parametrize("index_dtype", [torch.int64, torch.int32])
def test_decode_split_keys(device, d, index_dtype):
    _run(device, B=5, S=1, hq=8, hkv=2, d=d, L=1500, lens=[0, 1, 777, 1499, 64], causal=True,
         rows=[3, 0, 6, 1, 4], cache_rows=7, index_dtype=index_dtype)


@pytest.mark.parametrize("S,causal", [(3, True), (4, True), (4, False), (5, True)])
def test_short_chunks_around_the_decode_kernel(device, S, causal):
    """S * G <= 32 query rows per kv head take the decode kernel (each wave its own key tiles,
    merged through LDS), 40 rows the row-tile kernel; causal masks per token."""
    _run(device, B=3, S=S, hq=16, hkv=2, d=128, L=900, lens=[0, 451, 880], causal=causal, seed=20 + S)


def test_decode_uneven_rows(device):
    """Rows whose key ranges split into different numbers of parts (1 key to the whole cache)."""
    _run(device, B=8, S=1, hq=16, hkv=4, d=128, L=4096, lens=[0, 63, 64, 65, 1000, 4095, 2048, 129],
         causal=True, seed=5)


@pytest.mark.parametrize("causal", [True, False])
def test_chunked_prefill(device, causal):
    _run(device, B=3, S=100, hq=8, hkv=2, d=128, L=700, lens=[0, 37, 600], causal=causal, seed=1)


def test_prefill_mha_d64(device):
    _run(device, B=2, S=130, hq=4, hkv=4, d=64, L=400, lens=[5, 200], causal=True, seed=2)


def test_unsplit_launch(device):
    """Enough row tiles that the key range is not split (one workgroup per row tile)."""
    _run(device, B=4, S=1024, hq=16, hkv=4, d=128, L=1100, lens=[0, 3, 40, 76], causal=True, seed=3)


@pytest.mark.parametrize("validate", [True, False])
def test_validated_lengths(device, validate):
    """With validation the split is sized from the actual lengths; a write past the cache raises."""
    from mimir_amd import set_validate_metadata
    set_validate_metadata(validate)
    try:
        _run(device, B=3, S=1, hq=4, hkv=1, d=128, L=3000, lens=[10, 2000, 700], causal=True, seed=4)
        if validate:
            q = torch.zeros(1, 4, 2, 64, dtype=BF16, device=device)
            k = torch.zeros(1, 4, 2, 64, dtype=BF16, device=device)
            cache = Cache.create(1, 10, 2, 64, dtype=BF16, device=device)
            with pytest.raises(IndexError):
                attention_with_cache(q, k, k, cache, torch.tensor([7], device=device), True)
    finally:
        set_validate_metadata(False)


def test_rows_outside_the_cache_are_skipped(device):
    """Without validation a batch index outside the cache writes nothing and yields zeros."""
    gen = torch.Generator().manual_seed(9)
    q = torch.randn(2, 1, 4, 128, generator=gen).to(BF16).to(device)
    k = torch.randn(2, 1, 2, 128, generator=gen).to(BF16).to(device)
    cache = Cache(torch.randn(2, 64, 2, 128, generator=gen).to(BF16).to(device),
                  torch.randn(2, 64, 2, 128, generator=gen).to(BF16).to(device))
    before = cache.keys.clone()
    out = attention_with_cache(q, k, k, cache, torch.tensor([3, 5], device=device), True,
                               torch.tensor([1, 7], device=device))
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[1]) == 0 and torch.isfinite(out).all()
    assert torch.equal(cache.keys[0], before[0])
    # batch row 0 -> cache row 1, position cache_lengths[0] = 3
    assert torch.equal(cache.keys[1, 3], k[0, 0]) and torch.equal(cache.keys[1, :3], before[1, :3])
    assert torch.equal(cache.keys[1, 4:], before[1, 4:])


def test_repeated_calls_and_graph_replay(device):
    """The split arrival counters are cleared by each call: back-to-back calls and replays of a
    captured decode step (no host synchronisation, no memset) match the eager result."""
    gen = torch.Generator().manual_seed(11)
    B, hq, hkv, d, L = 4, 8, 2, 128, 2048
    q = torch.randn(B, 1, hq, d, generator=gen).to(BF16).to(device)
    k = torch.randn(B, 1, hkv, d, generator=gen).to(BF16).to(device)
    v = torch.randn(B, 1, hkv, d, generator=gen).to(BF16).to(device)
    cache = Cache(torch.randn(B, L, hkv, d, generator=gen).to(BF16).to(device),
                  torch.randn(B, L, hkv, d, generator=gen).to(BF16).to(device))
    lens = torch.tensor([5, 2000, 700, 1300], device=device)
    first = attention_with_cache(q, k, v, cache, lens, True)
    second = attention_with_cache(q, k, v, cache, lens, True)  # the same append again: same output
    torch.cuda.synchronize()
    assert torch.equal(first, second)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        attention_with_cache(q, k, v, cache, lens, True)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = attention_with_cache(q, k, v, cache, lens, True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        eager = attention_with_cache(q, k, v, cache, lens, True)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(eager, first)
