"""Seeded synthetic prefix-LM workloads and their work accounting.

The six measured shapes are the Mimir2 prefix-LM attention workloads:

1. fp32 forward, 4 x 512 tokens, 8 q-heads = 8 kv-heads, head_dim 64, prefix ~ U{0..512}
2. bf16 fwd+bwd, 8 x 2048 tokens, 16 q-heads / 4 kv-heads (GQA 4:1), head_dim 128, prefix ~ U{0..2048}
3. bf16 fwd+bwd, one packed row of 16384 tokens split into documents of length
   U{128..4096} (last truncated), prefix ~ U{0..L} per document, 16 / 4 heads, head_dim 128
4. bf16 fwd+bwd, 1 x 32768 tokens, 32 / 8 heads, head_dim 128, prefix 8192, one
   head_dim channel of q and k scaled x20 (softmax stress)
5. bf16 fwd+bwd, 64 x 1024 tokens, 8 / 8 heads, head_dim 64, prefix in {0, 1024}
6. bf16 fwd+bwd, the shape Mimir2's packaged sizes train at: multi-head attention
   (num_key_value_heads = num_heads, src/mimir/model/transformer.py:78) with the XXS
   size's 2 heads of 128 (src/mimir/conf/size/XXS.yaml:4-5, hidden 256), one packed row
   of 24576 tokens (global_batch_size 196608 / 8 ranks, src/mimir/conf/train.yaml:10)
   split into documents like workload 3 (the data config fixes no length law)

Inputs are drawn from a CPU ``torch.Generator`` in a fixed order -- q, k, v, dO
(standard normal, fp32) and then the metadata -- and cast to the compute dtype.
Metadata follows compute_aux_seq_tensors_scalars
(src/mimir/model/flash_attention_prefixlm_v2.py:21-35): int32 tensors padded to
the packed length and 0-d int64 CPU scalars (the training loop's convention,
src/mimir/training/loop.py:217).

Work accounting: a sequence of length n with prefix p has
N = (n^2 + n + p^2 - p) / 2 attended pairs; forward = 4*D*Hq*N FLOPs, backward =
10*D*Hq*N (2.5 x forward), masked pairs and recomputation never counted.
Compulsory HBM bytes: forward e*T*D*(2Hq + 2Hkv) + 4*T*Hq, backward
e*T*D*(4Hq + 4Hkv) + 12*T*Hq (e = element size).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch
from torch import Tensor

__all__ = ["Case", "CONFIG_NAMES", "bwd_bytes", "build_case", "fwd_bytes", "make_case", "make_config"]

CONFIG_NAMES = {
    1: "xxs_fp32_fwd_b4_s512_h8_d64",
    2: "gqa_bf16_b8_s2048_hq16_hkv4_d128",
    3: "packed_docs_bf16_t16384_hq16_hkv4_d128",
    4: "longctx_bf16_s32768_hq32_hkv8_d128_p8192_outlier20",
    5: "smallhead_bf16_b64_s1024_h8_d64_p0or1024",
    6: "xxs_mha_bf16_t24576_h2_d128_packed_docs",
}


@dataclass
class Case:
    q: Tensor
    k: Tensor
    v: Tensor
    dout: Tensor
    prefix_lens: Tensor       # int32 [max(T, numseqs + 1)], zero padded
    causal_lens: Tensor
    cu_seqlens: Tensor
    total_seqlen: Tensor      # 0-d int64 CPU tensors
    numseqs: Tensor
    max_seqlen_prefix: Tensor
    max_seqlen_causal: Tensor
    max_seqlen_all: Tensor
    is_causal: bool = False
    seq_lens: list = field(default_factory=list)
    prefixes: list = field(default_factory=list)
    meta: dict = field(default_factory=dict)

    @property
    def T(self) -> int:
        return self.q.shape[0]

    def call_args(self) -> tuple:
        """Positional metadata arguments of flash_attn_varlen_prefixlm after (q, k, v, is_causal)."""
        return (self.prefix_lens, self.causal_lens, self.cu_seqlens, self.total_seqlen, self.numseqs,
                self.max_seqlen_prefix, self.max_seqlen_causal, self.max_seqlen_all)

    def oracle_args(self) -> tuple:
        return (self.prefix_lens, self.causal_lens, self.cu_seqlens, self.total_seqlen, self.numseqs)

    def pairs(self) -> int:
        n = np.asarray(self.seq_lens, dtype=np.int64)
        p = np.zeros_like(n) if self.is_causal else np.asarray(self.prefixes, dtype=np.int64)
        return int(((n * n + n + p * p - p) // 2).sum())

    def fwd_flops(self) -> float:
        return 4.0 * self.q.shape[2] * self.q.shape[1] * self.pairs()

    def bwd_flops(self) -> float:
        return 10.0 * self.q.shape[2] * self.q.shape[1] * self.pairs()

    def to(self, device) -> "Case":
        mv = lambda t: t.to(device)
        return Case(mv(self.q), mv(self.k), mv(self.v), mv(self.dout), mv(self.prefix_lens),
                    mv(self.causal_lens), mv(self.cu_seqlens), self.total_seqlen, self.numseqs,
                    self.max_seqlen_prefix, self.max_seqlen_causal, self.max_seqlen_all, self.is_causal,
                    list(self.seq_lens), list(self.prefixes), dict(self.meta))


def fwd_bytes(T: int, hq: int, hkv: int, d: int, elem: int) -> float:
    return float(elem * T * d * (2 * hq + 2 * hkv) + 4 * T * hq)


def bwd_bytes(T: int, hq: int, hkv: int, d: int, elem: int) -> float:
    return float(elem * T * d * (4 * hq + 4 * hkv) + 12 * T * hq)


def draw_tensors(gen: torch.Generator, T: int, hq: int, hkv: int, d: int, dtype, outlier: float | None = None):
    q = torch.randn((T, hq, d), generator=gen)
    k = torch.randn((T, hkv, d), generator=gen)
    v = torch.randn((T, hkv, d), generator=gen)
    dout = torch.randn((T, hq, d), generator=gen)
    meta = {}
    if outlier is not None:
        ch = int(torch.randint(0, d, (1,), generator=gen).item())
        q[..., ch] *= outlier
        k[..., ch] *= outlier
        meta = {"outlier_channel": ch, "outlier_scale": float(outlier), "outlier_on": "q,k"}
    return (q.to(dtype), k.to(dtype), v.to(dtype), dout.to(dtype)), meta


def build_case(tensors, seq_lens, prefixes, *, is_causal: bool = False, meta: dict | None = None) -> Case:
    q, k, v, dout = tensors
    T = q.shape[0]
    seq_lens = [int(x) for x in seq_lens]
    prefixes = [int(x) for x in prefixes]
    nseq = len(seq_lens)
    total = sum(seq_lens)
    if total > T:
        raise ValueError("sequences exceed the packed length")
    padn = max(T, nseq + 1)
    pl = np.array(prefixes, dtype=np.int32)
    cl = np.array([n - p for n, p in zip(seq_lens, prefixes)], dtype=np.int32)
    cu = np.pad(np.cumsum(np.array(seq_lens, dtype=np.int64)).astype(np.int32), (1, padn - nseq - 1))
    pad = lambda a: torch.from_numpy(np.pad(a, (0, padn - a.shape[0])).astype(np.int32))
    scalar = lambda x: torch.tensor(int(x), dtype=torch.int64)
    return Case(
        q=q, k=k, v=v, dout=dout,
        prefix_lens=pad(pl), causal_lens=pad(cl), cu_seqlens=torch.from_numpy(cu.astype(np.int32)),
        total_seqlen=scalar(total), numseqs=scalar(nseq),
        max_seqlen_prefix=scalar(max(prefixes) if nseq else 0),
        max_seqlen_causal=scalar(int(cl.max()) if nseq else 0),
        max_seqlen_all=scalar(max(seq_lens) if nseq else 0),
        is_causal=is_causal, seq_lens=seq_lens, prefixes=prefixes, meta=dict(meta or {}),
    )


def make_case(seq_lens, prefixes, hq: int, hkv: int, d: int, *, seed: int = 0, dtype=torch.float32,
              pad_to: int | None = None, outlier: float | None = None, is_causal: bool = False) -> Case:
    """Small seeded case with explicit sequence and prefix lengths (padding rows if ``pad_to``)."""
    T = sum(int(x) for x in seq_lens) if pad_to is None else int(pad_to)
    gen = torch.Generator().manual_seed(seed)
    tensors, meta = draw_tensors(gen, T, hq, hkv, d, dtype, outlier)
    meta["seed"] = seed
    return build_case(tensors, seq_lens, prefixes, is_causal=is_causal, meta=meta)


def make_config(idx: int, seed: int = 0, dtype=None) -> Case:
    """One of the six measured workloads (see module docstring)."""
    gen = torch.Generator().manual_seed(seed)
    if idx == 1:
        T, hq, hkv, d, dt = 2048, 8, 8, 64, torch.float32
    elif idx in (2, 3):
        T, hq, hkv, d, dt = 16384, 16, 4, 128, torch.bfloat16
    elif idx == 4:
        T, hq, hkv, d, dt = 32768, 32, 8, 128, torch.bfloat16
    elif idx == 5:
        T, hq, hkv, d, dt = 65536, 8, 8, 64, torch.bfloat16
    elif idx == 6:
        T, hq, hkv, d, dt = 24576, 2, 2, 128, torch.bfloat16
    else:
        raise ValueError(f"unknown workload {idx}")
    dt = dtype or dt
    tensors, meta = draw_tensors(gen, T, hq, hkv, d, dt, 20.0 if idx == 4 else None)
    if idx == 1:
        seq_lens = [512] * 4
        prefixes = torch.randint(0, 513, (4,), generator=gen).tolist()
    elif idx == 2:
        seq_lens = [2048] * 8
        prefixes = torch.randint(0, 2049, (8,), generator=gen).tolist()
    elif idx in (3, 6):
        seq_lens, prefixes, left = [], [], T
        while left > 0:
            L = int(torch.randint(128, 4097, (1,), generator=gen).item())
            L = min(L, left)
            seq_lens.append(L)
            prefixes.append(int(torch.randint(0, L + 1, (1,), generator=gen).item()))
            left -= L
    elif idx == 4:
        seq_lens, prefixes = [32768], [8192]
    else:
        seq_lens = [1024] * 64
        prefixes = [1024 if b else 0 for b in (torch.rand(64, generator=gen) < 0.5).tolist()]
    meta.update({"seed": seed, "workload": CONFIG_NAMES[idx]})
    return build_case(tensors, seq_lens, prefixes, meta=meta)
