"""mimir_prefixlm_fwd_noalloc: the forward with its work list in the library's fixed
device array instead of a caller workspace, checked through the C ABI against
mimir_prefixlm_fwd on the same inputs (bitwise: the same kernels run over the same
work list; the array is far too small for the slots of the key-range parts, so the
workspace forward runs with a workspace that leaves them out too), on two calls in
a row, the second with a smaller input, and the refusal of a call whose work list
does not fit the array.  Collected last (the file name) so that a
failure here cannot hide the other GPU tests of a -x run."""

import ctypes

import pytest
import torch

from mimir_amd import _capi
from mimir_amd import prefixlm as P
from mimir_amd.workloads import make_case

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 128 * 1024  # the array's stated size: 8064 list entries of 16 bytes + 2 KiB K-scan slots
MAX_ENTRIES = (SCRATCH_BYTES - 2048) // 16


def _lib():
    return _capi.load()


def _forward(case, device, noalloc):
    c = case.to(device)
    lib = _lib()
    scale = 1.0 / case.q.shape[2] ** 0.5
    out_lo = torch.empty_like(c.q)
    saved = P._key_chunks
    P.set_key_chunks(False)  # the minimum workspace: no key-range parts
    try:
        p, out, lse, keep = P.prepare_fwd(c.q, c.k, c.v, case.is_causal, c.prefix_lens, c.causal_lens,
                                          c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_all, scale,
                                          out_lo=out_lo)
    finally:
        P._key_chunks = saved
    stream = torch.cuda.current_stream(device).cuda_stream
    if noalloc:
        p.workspace, p.workspace_bytes = None, 0  # the entry point brings its own
        rc = lib.mimir_prefixlm_fwd_noalloc(ctypes.byref(p), stream)
    else:
        rc = lib.mimir_prefixlm_fwd(ctypes.byref(p), stream)
    _capi.raise_for_status(lib, rc)
    torch.cuda.synchronize()
    return out.clone(), lse.clone(), out_lo.clone()


def test_noalloc_forward_matches_workspace_forward(device):
    big = make_case([1500, 700, 333, 45], [600, 0, 333, 10], 8, 2, 128, seed=61, dtype=torch.bfloat16, pad_to=2700)
    small = make_case([200, 64], [50, 64], 8, 2, 128, seed=62, dtype=torch.bfloat16)
    for label, case in (("first, larger", big), ("second, smaller", small)):
        ref = _forward(case, device, noalloc=False)
        got = _forward(case, device, noalloc=True)
        print(f"[noalloc] {label}: T={case.T} seqs={case.seq_lens}", flush=True)
        for a, b in zip(got, ref):
            assert torch.equal(a, b), label


def test_noalloc_refuses_a_work_list_beyond_its_array(device):
    lib = _lib()
    p = _capi.FwdParams()
    # the largest list that fits fills the array exactly
    assert lib.mimir_prefixlm_fwd_workspace_bytes(128 * (MAX_ENTRIES - 1), 1, 4096) == SCRATCH_BYTES
    p.total_tokens, p.numseqs, p.max_seqlen_all = 128 * MAX_ENTRIES, 1, 4096  # one entry more
    rc = lib.mimir_prefixlm_fwd_noalloc(ctypes.byref(p), None)
    assert rc == _capi.ERR_UNSUPPORTED_SHAPE
    assert b"131072-byte device array" in lib.mimir_prefixlm_last_error()
    with pytest.raises(ValueError):
        _capi.raise_for_status(lib, rc)
