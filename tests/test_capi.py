"""C ABI checks that need no GPU: the library loads, exports every entry point
include/mimir_prefixlm.h declares, the ctypes structs match the C layout, and
argument validation fails with the reference's exception types before any
device work is enqueued."""

import ctypes
import os
import re
import subprocess
import tempfile
from pathlib import Path

import pytest

from mimir_amd import _capi

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mimir_prefixlm.h"


@pytest.fixture(scope="module")
def lib():
    if not _capi.LIB_PATH.exists():
        from mimir_amd.build import build

        build(verbose=False)
    return _capi.load()


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\**\s+\**(mimir_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_the_binding_symbols():
    assert declared_functions() == sorted(_capi.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_capi.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for sym in declared_functions():
        assert sym in exported, sym
        getattr(lib, sym)


def test_abi_version(lib):
    assert lib.mimir_prefixlm_abi_version() == _capi.ABI_VERSION


def _align256(x):
    return (x + 255) // 256 * 256


def _fwd_workspace(T, numseqs):
    """Forward workspace: the tile list, one int4 per entry, ceil(T / 128) + numseqs entries
    (max_seqlen_all unused), then 256-byte aligned the 512 int32 K-scan slots."""
    cap = -(-T // 128) + numseqs
    return _align256(cap * 16) + 512 * 4


def _fwd_workspace_chunked(T, numseqs, hq, d):
    """With key-range parts: 1024 // hq chunk slots more list entries, then 256-byte aligned
    the K-scan slots, one int32 arrival counter per (slot, q head), and per (slot, q head)
    the partial O (fp32, d x 128) plus running max and sum of 64 lanes x 4 waves."""
    slots = 1024 // hq
    cap = -(-T // 128) + numseqs + slots
    ctr = _align256(_align256(cap * 16) + 512 * 4)
    part = _align256(ctr + slots * hq * 4)
    return part + slots * hq * (4 * d * 128 + 4 * 64 * 8)


@pytest.mark.parametrize("T,total,ns,hq,d,dtype,chunked", [
    (24576, 24576, 11, 2, 128, _capi.DTYPE_BFLOAT16, True),     # 192 tiles x 2 heads < 512
    (24576, 24576, 11, 2, 64, _capi.DTYPE_BFLOAT16, True),
    (255 * 128, 255 * 128, 3, 2, 128, _capi.DTYPE_BFLOAT16, True),  # 255 x 2 = 510
    (256 * 128, 256 * 128, 3, 2, 128, _capi.DTYPE_BFLOAT16, False),  # 256 x 2 = 512: cannot be small
    (256 * 128, 3000, 3, 2, 128, _capi.DTYPE_BFLOAT16, True),  # padded: 3000 real tokens, 24 x 2 tiles
    (256 * 128, 0, 3, 2, 128, _capi.DTYPE_BFLOAT16, False),    # no active token: nothing to cut
    (16384, 16384, 8, 16, 128, _capi.DTYPE_BFLOAT16, False),
    (24576, 24576, 11, 2, 128, _capi.DTYPE_FLOAT32, False),
    (0, 0, 0, 2, 128, _capi.DTYPE_BFLOAT16, False),
])
def test_fwd_workspace_size(lib, T, total, ns, hq, d, dtype, chunked):
    """The chunk room is sized where the grid can be small: ceil(min(T, total_seqlen) / 128) x Hq < 512."""
    p = _capi.FwdParams()
    p.total_tokens, p.numseqs, p.max_seqlen_all, p.num_q_heads, p.head_dim, p.dtype = T, ns, 4096, hq, d, dtype
    p.total_seqlen = total
    got = lib.mimir_prefixlm_fwd_workspace_size(ctypes.byref(p))
    base = lib.mimir_prefixlm_fwd_workspace_bytes(T, ns, 4096)
    assert got == (_fwd_workspace_chunked(T, ns, hq, d) if chunked else base), (got, base)
    assert lib.mimir_prefixlm_fwd_workspace_size(None) == 0


def test_workspace_bytes(lib):
    for T, ns, mx in ((16384, 8, 2048), (16384, 8, 100), (16384, 1000, 4096), (5, 1, 5)):
        assert lib.mimir_prefixlm_fwd_workspace_bytes(T, ns, mx) == _fwd_workspace(T, ns), (T, ns, mx)
    assert lib.mimir_prefixlm_fwd_workspace_bytes(0, 8, 2048) == 0
    for args in ((16384, 16, 8, 2048), (2048, 8, 4, 512), (16384, 16, 1000, 4096), (100, 3, 1, 100)):
        assert lib.mimir_prefixlm_bwd_workspace_bytes(*args) == _bwd_workspace(*args), args
    assert lib.mimir_prefixlm_bwd_workspace_bytes(0, 16, 8, 2048) == 0


def _bwd_workspace(T, hq, numseqs, max_len):
    """Backward workspace: 256-byte aligned sections delta and lse*log2(e) (float32 [Hq, T]), the
    query-tile list (int4 per tile), the key-tile list (int4 per tile plus one per possible split pair),
    one int32 counter per split (pair, kv head) plus two work-queue counters and the dS-incomplete flag,
    512 int32 K-scan slots, and two float32 slots of 2 * 128 * 128 per split (pair, kv head)."""
    def align(x):
        return (x + 255) // 256 * 256
    cap = -(-T // 128) + numseqs
    pair_heads = min(384, cap * hq)
    lse2 = align(T * hq * 4)
    plan_q = align(lse2 + T * hq * 4)
    plan_k = align(plan_q + cap * 16)
    counters = align(plan_k + (cap + pair_heads) * 16)
    kscan = align(counters + (pair_heads + 3) * 4)
    slots = align(kscan + 512 * 4)
    return slots + pair_heads * 2 * 2 * 128 * 128 * 4


@pytest.mark.parametrize("T,total,ns,hq,d,dtype,chunked", [
    (24576, 24576, 11, 2, 128, _capi.DTYPE_BFLOAT16, True),
    (24576, 24576, 11, 2, 64, _capi.DTYPE_BFLOAT16, True),
    (256 * 128, 256 * 128, 3, 2, 128, _capi.DTYPE_BFLOAT16, False),  # the grid cannot be small
    (256 * 128, 3000, 3, 2, 128, _capi.DTYPE_BFLOAT16, True),        # padded: 3000 real tokens
    (24576, 24576, 11, 2, 128, _capi.DTYPE_FLOAT32, False),
])
def test_bwd_workspace_with_dq_chunks(lib, T, total, ns, hq, d, dtype, chunked):
    """dq_key_chunks adds, after the rest of the workspace, the dQ list with room for the parts
    (int4 [cap + 1024 // hq]), one int32 counter per (chunk slot, q head) and the chunk slots;
    only where the grid can be small (ceil(min(T, total_seqlen) / 128) * hq < 512) and for bf16."""
    def align(x):
        return (x + 255) // 256 * 256
    p = _capi.BwdParams()
    p.total_tokens, p.num_q_heads, p.num_kv_heads, p.numseqs, p.max_seqlen_all = T, hq, hq, ns, 4096
    p.total_seqlen = total
    p.head_dim, p.dtype = d, dtype
    base = lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p))
    assert base == _bwd_workspace(T, hq, ns, 4096)
    p.dq_key_chunks = 1
    got = lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p))
    if not chunked:
        assert got == base
        return
    slots = 1024 // hq
    cap = -(-T // 128) + ns
    ctr = align(align(base) + (cap + slots) * 16)
    part = align(ctr + slots * hq * 4)
    assert got == part + slots * hq * (4 * d * 128 + 4 * 64 * 8)


def test_tile_list_capacity_covers_every_packing(lib):
    """The list capacity ceil(T / 128) + numseqs bounds sum_s ceil(n_s / 128) for every packing of at
    most T tokens into numseqs sequences, whatever max_seqlen_all says: random packings, all-equal,
    one long sequence plus empties, and lengths of 128 k + 1 (the worst case of the ceilings)."""
    import numpy as np

    rng = np.random.default_rng(0)
    packings = [[128 * 3 + 1] * 40, [16384] + [0] * 7, [1] * 300, [2048] * 8, [129] * 100]
    for _ in range(200):
        ns = int(rng.integers(1, 60))
        cuts = np.sort(rng.integers(0, 20000, ns - 1))
        packings.append(np.diff(np.concatenate([[0], cuts, [int(rng.integers(cuts[-1] if ns > 1 else 0, 20001))]]))
                        .tolist())
    for lens in packings:
        T, ns = int(sum(lens)) + int(rng.integers(0, 200)), len(lens)
        if T == 0:
            continue
        tiles = sum(-(-n // 128) for n in lens)
        cap = -(-T // 128) + ns
        assert tiles <= cap, (lens[:5], T, ns, tiles, cap)
        for claimed_max in (1, max(lens) if max(lens) > 0 else 1):  # an understated max changes nothing
            assert lib.mimir_prefixlm_fwd_workspace_bytes(T, ns, claimed_max) == _fwd_workspace(T, ns)


def _c_layout(struct_name, fields):
    """offsetof / sizeof of a header struct, from a C program built with gcc."""
    src = '#include <stdio.h>\n#include <stddef.h>\n#include "mimir_prefixlm.h"\nint main(void){\n'
    src += f'printf("%zu\\n", sizeof({struct_name}));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof({struct_name}, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "layout.c")
        exe = os.path.join(d, "layout")
        with open(c, "w") as fh:
            fh.write(src)
        subprocess.run(["gcc", "-I", str(HEADER.parent), c, "-o", exe], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    return vals[0], vals[1:]


@pytest.mark.parametrize("cls,name", [(_capi.FwdParams, "MimirPrefixLMFwdParams"),
                                      (_capi.BwdParams, "MimirPrefixLMBwdParams"),
                                      (_capi.RopeParams, "MimirRopeParams"),
                                      (_capi.CacheAttnParams, "MimirCacheAttnParams")])
def test_ctypes_struct_matches_c_layout(cls, name):
    fields = [f for f, _ in cls._fields_]
    size, offsets = _c_layout(name, fields)
    assert ctypes.sizeof(cls) == size
    assert [getattr(cls, f).offset for f in fields] == offsets


def test_null_params_is_invalid_argument(lib):
    assert lib.mimir_prefixlm_fwd(None, None) == _capi.ERR_INVALID_ARGUMENT
    assert b"NULL" in lib.mimir_prefixlm_last_error()
    assert lib.mimir_prefixlm_bwd(None, None) == _capi.ERR_INVALID_ARGUMENT


def _fwd(**kw):
    p = _capi.FwdParams()
    base = dict(total_tokens=16, num_q_heads=4, num_kv_heads=2, head_dim=128, numseqs=1, total_seqlen=16,
                max_seqlen_all=16, dtype=_capi.DTYPE_BFLOAT16, softmax_scale=0.088)
    base.update(kw)
    for k, v in base.items():
        setattr(p, k, v)
    return p


def test_validation_errors_map_to_reference_exceptions(lib):
    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd(num_q_heads=3)), None)
    assert rc == _capi.ERR_INVALID_ARGUMENT
    assert b"Query heads 3 must be divisible by key/value heads 2." in lib.mimir_prefixlm_last_error()
    with pytest.raises(ValueError, match="divisible"):
        _capi.raise_for_status(lib, rc)

    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd(dtype=7)), None)
    assert rc == _capi.ERR_UNSUPPORTED_DTYPE
    with pytest.raises(TypeError):
        _capi.raise_for_status(lib, rc)

    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd(head_dim=96)), None)
    assert rc == _capi.ERR_UNSUPPORTED_SHAPE
    assert b"head_dim 96" in lib.mimir_prefixlm_last_error()

    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd(total_seqlen=17)), None)
    assert rc == _capi.ERR_INVALID_ARGUMENT

    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd(softmax_scale=0.0)), None)
    assert rc == _capi.ERR_INVALID_ARGUMENT

    # q is NULL: rejected before any launch
    rc = lib.mimir_prefixlm_fwd(ctypes.byref(_fwd()), None)
    assert rc == _capi.ERR_INVALID_ARGUMENT and b"q is NULL" in lib.mimir_prefixlm_last_error()


def test_dscore_workspace_bytes(lib):
    """The score-gradient hand-off: Hq x (T/32 + numseqs + 1) x ceil(max_seqlen/32) blocks of
    2 KiB, only for bf16 with head_dim 128 and only within dscore_limit_bytes; the workspace
    grows by exactly that (after 256-byte alignment)."""
    p = _capi.BwdParams()
    p.total_tokens, p.num_q_heads, p.num_kv_heads, p.numseqs, p.max_seqlen_all = 1000, 8, 2, 3, 700
    p.head_dim, p.dtype = 128, _capi.DTYPE_BFLOAT16
    expect = 8 * (1000 // 32 + 3 + 1) * ((700 + 31) // 32) * 2048
    p.dscore_limit_bytes = 0
    assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == 0
    base = lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p))
    assert base == lib.mimir_prefixlm_bwd_workspace_bytes(1000, 8, 3, 700)
    for limit, got in ((expect - 1, 0), (expect, expect), (1 << 40, expect)):
        p.dscore_limit_bytes = limit
        assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == got
        size = lib.mimir_prefixlm_bwd_workspace_size(ctypes.byref(p))
        assert size == (base if got == 0 else ((base + 255) // 256) * 256 + expect)
    p.split_mode = _capi.SPLIT_ALWAYS  # the stored tiles have no low half: no hand-off
    assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == 0
    p.split_mode = _capi.SPLIT_NEVER
    assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == expect
    p.split_mode = _capi.SPLIT_AUTO
    p.head_dim = 64
    assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == 0
    p.head_dim, p.dtype = 128, _capi.DTYPE_FLOAT32
    assert lib.mimir_prefixlm_bwd_dscore_bytes(ctypes.byref(p)) == 0


def test_low_half_and_split_mode_validation(lib):
    """out_lo is a bf16-only operand (forward and backward); split_mode must be a known mode.
    Both are rejected before any launch (the tensors here are NULL / fake addresses)."""
    p = _fwd(dtype=_capi.DTYPE_FLOAT32, q=16, k=16, v=16, out=16, q_stride_token=512, q_stride_head=128,
             k_stride_token=256, k_stride_head=128, v_stride_token=256, v_stride_head=128, out_stride_token=512,
             out_stride_head=128, prefix_lens=16, cu_seqlens=16, workspace=16, workspace_bytes=1 << 20,
             out_lo=16, out_lo_stride_token=512, out_lo_stride_head=128)
    assert lib.mimir_prefixlm_fwd(ctypes.byref(p), None) == _capi.ERR_INVALID_ARGUMENT
    assert b"out_lo" in lib.mimir_prefixlm_last_error()
    b = _capi.BwdParams()
    for f, v in dict(total_tokens=16, num_q_heads=4, num_kv_heads=2, head_dim=128, numseqs=1, total_seqlen=16,
                     max_seqlen_all=16, dtype=_capi.DTYPE_BFLOAT16, softmax_scale=0.088, lse_stride_head=16,
                     prefix_lens=16, cu_seqlens=16, lse=16).items():
        setattr(b, f, v)
    for name in ("q", "k", "v", "out", "dout", "dq", "dk", "dv"):
        heads = 4 if name in ("q", "out", "dout", "dq") else 2
        setattr(b, name, 16)
        setattr(b, name + "_stride_token", heads * 128)
        setattr(b, name + "_stride_head", 128)
    b.split_mode = 3
    assert lib.mimir_prefixlm_bwd(ctypes.byref(b), None) == _capi.ERR_INVALID_ARGUMENT
    assert b"split_mode" in lib.mimir_prefixlm_last_error()


def test_rope_table_validation(lib):
    """RoPE inside the kernels: bf16 only, cos and sin together, aligned float32 rows of at least
    head_dim, and q_rope only with the tables.  All rejected before any launch."""
    ops = dict(q=16, k=16, v=16, out=16, q_stride_token=512, q_stride_head=128, k_stride_token=256,
               k_stride_head=128, v_stride_token=256, v_stride_head=128, out_stride_token=512, out_stride_head=128,
               prefix_lens=16, cu_seqlens=16, workspace=16, workspace_bytes=1 << 20)
    cases = [
        (dict(dtype=_capi.DTYPE_FLOAT32, rope_cos=16, rope_sin=32, rope_stride_token=128),
         _capi.ERR_UNSUPPORTED_DTYPE, b"bfloat16 only"),
        (dict(rope_cos=16, rope_stride_token=128), _capi.ERR_INVALID_ARGUMENT, b"go together"),
        (dict(rope_cos=16, rope_sin=36, rope_stride_token=128), _capi.ERR_INVALID_ARGUMENT, b"16-byte aligned"),
        (dict(rope_cos=16, rope_sin=32, rope_stride_token=64), _capi.ERR_INVALID_ARGUMENT, b"at least head_dim"),
        (dict(rope_cos=16, rope_sin=32, rope_stride_token=130), _capi.ERR_INVALID_ARGUMENT, b"multiple of 4"),
        (dict(q_rope=16, q_rope_stride_token=512, q_rope_stride_head=128), _capi.ERR_INVALID_ARGUMENT,
         b"q_rope needs"),
    ]
    for extra, code, msg in cases:
        p = _fwd(**ops, **extra)
        assert lib.mimir_prefixlm_fwd(ctypes.byref(p), None) == code, extra
        assert msg in lib.mimir_prefixlm_last_error(), (extra, lib.mimir_prefixlm_last_error())


def test_unknown_backward_stage_bits(lib):
    p = _capi.BwdParams()
    assert lib.mimir_prefixlm_bwd_stages(ctypes.byref(p), 64, None) == _capi.ERR_INVALID_ARGUMENT


def test_last_error_is_thread_local(lib):
    import threading

    lib.mimir_prefixlm_fwd(None, None)
    seen = []

    def worker():
        seen.append(lib.mimir_prefixlm_last_error())

    t = threading.Thread(target=worker)
    t.start()
    t.join()
    assert seen == [b""]
    assert lib.mimir_prefixlm_last_error() != b""
