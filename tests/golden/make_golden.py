"""Write the golden prefix-LM fixtures (tests/golden/*.npz).

The reference ships no golden vectors for its attention operator, so these are
computed here by explicit fp64 loops over (query, head, key) using the Metal
mask predicate (oracle.prefixlm_oracle.brute_force_forward / _backward), on
seeded inputs rounded to bfloat16 so that the same file checks the bf16 and the
fp32 kernels.  Regenerate with:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from mimir_amd.workloads import make_case  # noqa: E402
from oracle.prefixlm_oracle import brute_force_backward, brute_force_forward  # noqa: E402

CASES = {
    "packed_gqa_d64": dict(seq_lens=[40, 24, 17], prefixes=[13, 24, 0], hq=4, hkv=2, d=64, pad_to=96, causal=False),
    "bidir_d128": dict(seq_lens=[70], prefixes=[70], hq=2, hkv=1, d=128, pad_to=None, causal=False),
    "causal_d64": dict(seq_lens=[33, 30], prefixes=[5, 29], hq=2, hkv=2, d=64, pad_to=None, causal=True),
}


def main():
    for i, (name, cfg) in enumerate(CASES.items()):
        c = make_case(cfg["seq_lens"], cfg["prefixes"], cfg["hq"], cfg["hkv"], cfg["d"], seed=1000 + i,
                      dtype=torch.bfloat16, pad_to=cfg["pad_to"], is_causal=cfg["causal"])
        q, k, v, do = (t.float() for t in (c.q, c.k, c.v, c.dout))
        args = c.oracle_args()
        o, lse = brute_force_forward(q, k, v, c.is_causal, *args)
        dq, dk, dv = brute_force_backward(q, k, v, do, c.is_causal, *args)
        np.savez_compressed(
            os.path.join(HERE, f"{name}.npz"),
            q=q.numpy(), k=k.numpy(), v=v.numpy(), dout=do.numpy(),
            prefix_lens=c.prefix_lens.numpy(), causal_lens=c.causal_lens.numpy(), cu_seqlens=c.cu_seqlens.numpy(),
            total_seqlen=np.int64(int(c.total_seqlen)), numseqs=np.int64(int(c.numseqs)),
            max_seqlen_all=np.int64(int(c.max_seqlen_all)), is_causal=np.bool_(c.is_causal),
            o=o, lse=lse, dq=dq, dk=dk, dv=dv,
        )
        print("wrote", name)


if __name__ == "__main__":
    main()
