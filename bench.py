#!/usr/bin/env python3
"""Prefix-LM attention forward+backward throughput on one MI355X.

One step = one forward and one backward pass of the prefix-LM attention
operator over one packed batch, with every input already resident in HBM:
``mimir_prefixlm_fwd`` followed by ``mimir_prefixlm_bwd`` (delta, dK/dV, dQ,
padding fill), all through the C ABI on torch's current stream.  The default workload is 8 sequences x 2048 tokens,
16 q-heads / 4 kv-heads (GQA), head_dim 128, bf16, prefix lengths ~ U{0..2048}
(seed 0).

``value`` counts only attended (unmasked) pairs: fwd 4*D*Hq*N, bwd 10*D*Hq*N
FLOPs with N = sum over sequences of (n^2 + n + p^2 - p)/2.  The roofline entry
is for the kernel that takes the most time; its algorithmic FLOPs per launch are
fwd 4*D*Hq*N, dK/dV 8*D*Hq*N (S recompute, dP, dV, dK) and dQ 2*D*Hq*N (dQ only;
when dQ recomputes S and dP, that is not counted), so the three add up to the
step's 14*D*Hq*N.  With the score-gradient hand-off (bf16, head_dim 128) the dQ
kernel reads the dS blocks the dK/dV kernel stored; the line then also gives its
streamed bytes and bandwidth (``dq_ds_bytes``, ``dq_ds_gbs``).
Timing: after a warm-up of at least ``--warmup`` steps and ``--warmup-seconds``
(so the clocks settle), the timed region runs K steps back to back between two
HIP events on the launch stream; ``value`` and ``ms_per_step`` come from it.  A
second pass of K steps records an event at every step boundary for the per-step
median, a third times the forward alone, and a fourth runs the stages serialized
(``mimir_prefixlm_bwd_stages``) with events between them for the per-kernel
durations the roofline entry uses.  The CPU baseline times the oracle's restatement of the reference
masked-SDPA path (fp32, autograd) on a bounded sample of the same batch.

Prints exactly one JSON line.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

PEAK_BF16_TFLOPS = 2516.6   # 256 CU x 2.4 GHz x 4096 FLOP/clk, dense
PEAK_F32_TFLOPS = 157.3     # fp32 matrix
HBM_GBS = 8000.0
METRIC = "prefix-LM attn fwd+bwd TFLOP/s (unmasked) bf16, % of MI355X MFMA peak"


def _cores() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(case, target_seconds: float = 4.0, unit_bytes_cap: float = 3e9, runs: int = 3) -> dict:
    """Oracle masked-SDPA fwd+bwd and fwd alone (fp32, autograd) over a bounded sample of the batch.

    The sample is a fixed round-robin list of units = (sequence, range of q-heads),
    each run densely as its own packed batch: as many units as one fwd+bwd pass
    covers in about ``target_seconds`` (after one untimed warm-up unit).  A unit
    holds as many whole kv-head groups as fit in ``unit_bytes_cap`` of fp32 score
    matrices, or fewer q-heads of one group when a single group does not fit.
    The sample is then timed ``runs`` times fwd+bwd and ``runs`` times forward
    only; the medians are reported.  FLOPs count the units' attended pairs
    only, like the GPU figure.
    """
    import torch

    from oracle.prefixlm_oracle import dense_forward_autograd
    from mimir_amd.workloads import build_case

    cores = _cores()
    torch.set_num_threads(cores)
    hq, hkv = case.q.shape[1], case.k.shape[1]
    group = hq // hkv
    units = []   # (sequence, first q-head, q-heads, first kv head, kv heads)
    for si, n in enumerate(case.seq_lens):
        fit = max(1, int(unit_bytes_cap // (6.0 * 4.0 * n * n)))   # scores, probabilities, their grads
        if fit >= group:
            kv_w = max(d_ for d_ in range(1, hkv + 1) if hkv % d_ == 0 and d_ * group <= fit)
            units += [(si, kv0 * group, kv_w * group, kv0, kv_w) for kv0 in range(0, hkv, kv_w)]
        else:
            w = max(d_ for d_ in range(1, group + 1) if group % d_ == 0 and d_ <= fit)
            units += [(si, q0, w, q0 // group, 1) for q0 in range(0, hq, w)]

    def make(unit):
        si, q0, qw, kv0, kvw = unit
        n, p = case.seq_lens[si], case.prefixes[si]
        s0 = int(case.cu_seqlens[si])
        sl = slice(s0, s0 + n)
        tens = (case.q[sl, q0:q0 + qw].float().contiguous(), case.k[sl, kv0:kv0 + kvw].float().contiguous(),
                case.v[sl, kv0:kv0 + kvw].float().contiguous(), case.dout[sl, q0:q0 + qw].float().contiguous())
        return build_case(tens, [n], [p], is_causal=case.is_causal)

    def run(sample, backward=True):
        q, k, v = (t.clone().requires_grad_(backward) for t in (sample.q, sample.k, sample.v))
        if backward:
            dense_forward_autograd(q, k, v, sample.is_causal, *sample.oracle_args()).backward(sample.dout)
        else:
            with torch.no_grad():
                dense_forward_autograd(q, k, v, sample.is_causal, *sample.oracle_args())

    run(make(units[0]))  # warm-up
    chosen = []  # the sample: units until one fwd+bwd pass takes target_seconds
    elapsed = 0.0
    while elapsed < target_seconds:
        sample = make(units[len(chosen) % len(units)])
        t0 = time.perf_counter()
        run(sample)
        elapsed += time.perf_counter() - t0
        chosen.append(sample)
    flops_fwd = sum(s.fwd_flops() for s in chosen)
    flops = flops_fwd + sum(s.bwd_flops() for s in chosen)

    def timed(backward):
        t0 = time.perf_counter()
        for smp in chosen:
            run(smp, backward)
        return time.perf_counter() - t0

    t_step = statistics.median(timed(True) for _ in range(runs))
    t_fwd = statistics.median(timed(False) for _ in range(runs))
    done = len(chosen)
    try:
        model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name"))
    except Exception:  # noqa: BLE001
        model = "unknown"
    widths = sorted({u[2] for u in units})
    return {
        "value": round(flops / t_step / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"{done} units of (sequence, {'/'.join(map(str, widths))} q-heads) of the "
                   f"same batch ({len(units)} units cover it; round-robin from sequence 0), each fwd+bwd as fp32 "
                   f"torch SDPA with a bool prefix-LM mask + autograd; median of {runs} timed passes over the "
                   f"sample after 1 warm-up unit"),
        "seconds": round(t_step, 3),
        "fwd_value": round(flops_fwd / t_fwd / 1e12, 5),
        "fwd_seconds": round(t_fwd, 3),
        "runs": runs,
        "cpu_model": model,
        "torch": torch.__version__,
    }


def dscore_blocks(case) -> int:
    """32 x 32 (query, key) blocks per head holding at least one attended pair: the dS
    blocks the dK / dV kernel stores and the dQ kernel reads with the score-gradient hand-off."""
    cu = case.cu_seqlens.tolist()
    pl = case.prefix_lens.tolist()
    total = 0
    for s in range(int(case.numseqs)):
        n = cu[s + 1] - cu[s]
        p = 0 if case.is_causal else min(max(pl[s], 0), n)
        for qa in range(0, n, 32):
            total += (max(p, min(qa + 32, n)) + 31) // 32
    return total


def auto_split(case, scale: float) -> bool:
    """The device-side AUTO rule (softmax_scale * max|K| > 0.75 over the keys inside
    sequences) on the host copy of K: whether the bf16 kernels carry P and dS split."""
    if case.k.element_size() != 2:
        return False
    cu = case.cu_seqlens.tolist()
    keys = case.k[cu[0]:cu[int(case.numseqs)]]
    return keys.numel() > 0 and bool(keys.float().abs().max().item() * scale > 0.75)


def working_kernels(d: int, elem: int, handoff: bool) -> dict:
    """Full names, as rocprofv3 reports them, of the kernels that do each stage's work.

    One bf16 kernel serves both split modes (the device-side decision picks the
    body inside it).  ``handoff``: the dK/dV kernel stores dS and dq_ds_kernel
    reads it.
    """
    if elem == 4:
        return {"fwd": f"fwd_f32_kernel<{d}>", "dkdv": f"dkdv_f32_kernel<{d}>", "dq": f"dq_f32_kernel<{d}>"}
    if d == 128:
        dkdv = "dkdv_pair_ds_kernel" if handoff else "dkdv_pair_kernel"
    else:
        dkdv = f"dkdv_kernel<{d}>"
    return {"fwd": f"fwd_bf16_kernel<{d}>", "dkdv": dkdv, "dq": "dq_ds_kernel" if handoff else f"dq_kernel<{d}>"}


def _measured_traffic(workload: str, kernel: str):
    """HBM bytes per launch of ``kernel`` (full instantiation name) on ``workload``.

    profiles/hbm_traffic.json holds FETCH_SIZE and WRITE_SIZE per dispatch from two
    rocprofv3 --pmc runs of this script, each scaled by what the same counter reads
    for a plain 1 GiB device copy, keyed by the full instantiation name (the plain
    and split bodies share one kernel, so a workload holds one entry per stage); None when the
    workload or the kernel was not profiled.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as fh:
            data = json.load(fh)
        entry = data["workloads"][workload][kernel]
    except (OSError, KeyError, ValueError):
        return None
    cal = data["calibration"]
    return {"bytes": int(entry["bytes"]),
            "source": (f"profiles/hbm_traffic.json (tree {data.get('commit', '?')}): FETCH_SIZE {entry['fetch_kib']} KiB x "
                       f"{cal['fetch_factor']} + WRITE_SIZE {entry['write_kib']} KiB x {cal['write_factor']}, factors "
                       f"from a 1 GiB device copy")}


def copy_calibration(torch, dev, mib: int, reps: int) -> int:
    """Copy ``mib`` MiB device-to-device ``reps`` times: each launch reads and writes exactly mib MiB."""
    n = mib * (1 << 20) // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    print(json.dumps({"copy_mib": mib, "bytes_read": n * 4, "bytes_written": n * 4, "launches": reps + 1,
                      "ms_per_copy": round(ms, 5), "gbs_read_plus_write": round(2 * n * 4 / ms / 1e6, 1)}), flush=True)
    return 0


def layer_bench(torch, dev, args) -> int:
    """The attention layer core of src/mimir/model/layers.py:182-239 on a workload's shapes.

    fused:   mimir_amd.layer.gated_attention (bf16: q rotated inside the attention
             forward, which also writes the rotated copy the backward streams, k by
             one RoPE kernel pass, dQ / dK mapped back in the backward's stores; the
             gate in the attention store and its backward in the delta rows; one gqkv
             gradient)
    unfused: the reference's composition -- split views, fp32 torch RoPE
             (layers.py:24-40), the same prefix-LM operator, torch.sigmoid(gate) * attn
    Both run forward + backward from the gqkv projection output to the o_proj input.
    The RoPE kernel is also timed alone against the HBM roofline (bytes: q read and
    written, cos / sin read).  Prints one JSON line.
    """
    from mimir_amd import flash_attn_varlen_prefixlm
    from mimir_amd import layer as L
    from mimir_amd.workloads import CONFIG_NAMES, make_config

    case = make_config(args.workload, seed=args.seed)
    c = case.to(dev)
    T, hq, d = case.q.shape
    hkv = case.k.shape[1]
    dt = case.q.dtype
    gen = torch.Generator().manual_seed(args.seed + 1)
    gqkv = torch.randn(T, (2 * hq + 2 * hkv) * d, generator=gen).to(dt).to(dev)
    dy = torch.randn(T, hq * d, generator=gen).to(dt).to(dev)
    pos = torch.cat([torch.arange(n) for n in case.seq_lens] + [torch.zeros(T - sum(case.seq_lens), dtype=torch.int64)])
    inv_freq = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    emb = torch.cat((torch.outer(pos.float(), inv_freq),) * 2, dim=-1)
    cos, sin = emb.cos().to(dev), emb.sin().to(dev)
    meta = dict(prefix_lens=c.prefix_lens, causal_lens=c.causal_lens, cu_seqlens=c.cu_seqlens,
                total_seqlen=c.total_seqlen, numseqs=c.numseqs, max_seqlen_all=c.max_seqlen_all)

    def rope_torch(x):
        x1, x2 = x[..., : d // 2], x[..., d // 2:]
        return ((x * cos.unsqueeze(-2)) + (torch.cat((-x2, x1), dim=-1) * sin.unsqueeze(-2))).to(x.dtype)

    def fused():
        g = gqkv.detach().requires_grad_(True)
        L.gated_attention(g, (cos, sin), hq, hkv, case.is_causal, **meta).backward(dy)

    def unfused():
        g = gqkv.detach().requires_grad_(True)
        gate, q, k, v = g.view(T, 2 * hq + 2 * hkv, d).split((hq, hq, hkv, hkv), dim=1)
        attn = flash_attn_varlen_prefixlm(rope_torch(q), rope_torch(k), v, case.is_causal,
                                          max_seqlen_prefix=c.max_seqlen_prefix,
                                          max_seqlen_causal=c.max_seqlen_causal, **meta)
        (torch.sigmoid(gate) * attn).reshape(T, hq * d).backward(dy)

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    K, W = max(1, args.steps), max(1, args.warmup)
    ms_fused = timed(fused, K, W)
    ms_unfused = timed(unfused, K, W)
    qv = gqkv.view(T, 2 * hq + 2 * hkv, d)[:, hq:2 * hq]
    out = torch.empty((T, hq, d), dtype=dt, device=dev)
    ms_rope = timed(lambda: L.rope(qv, cos, sin, out=out), 4 * K, W)
    rope_bytes = 2 * T * hq * d * gqkv.element_size() + 2 * T * d * 4
    rope_gbs = rope_bytes / (ms_rope * 1e-3) / 1e9
    res = {
        "metric": "attention layer core (split, RoPE, prefix-LM attention, sigmoid gate) fwd+bwd ms",
        "value": round(ms_fused, 4),
        "unit": "ms",
        "higher_is_better": False,
        "steps": K,
        "warmup": W,
        "dtype": "bf16" if dt == torch.bfloat16 else "fp32",
        "data": "synthetic",
        "config": {"workload": CONFIG_NAMES[args.workload], "tokens": T, "q_heads": hq, "kv_heads": hkv,
                   "head_dim": d, "gqkv_shape": [T, (2 * hq + 2 * hkv) * d], "seed": args.seed},
        "unfused_ms": round(ms_unfused, 4),
        "speedup_vs_unfused": round(ms_unfused / ms_fused, 3),
        "rope": {"kernel": "rope_kernel", "ms": round(ms_rope, 5), "bound": "hbm", "achieved": round(rope_gbs, 1),
                 "peak": HBM_GBS, "unit": "GB/s", "frac": round(rope_gbs / HBM_GBS, 4),
                 "bytes_per_launch": rope_bytes},
    }
    print(json.dumps(res), flush=True)
    return 0


def cache_bench(torch, dev, args) -> int:
    """KV-cache attention (src/mimir/model/layers.py:134-167) at the default workload's heads.

    decode:  B = 8 rows, one new token each, cache lengths ~ U{1024..4096} (seed), L = 4096;
             bound by reading the cache: bytes = sum_b kv_len_b * Hkv * D * 2 (K and V) * 2 B
             plus q, out and the appended rows.
    prefill: the same rows take a 512-token chunk on top of 1536 cached tokens (causal).
    The reference composition (cache scatter, repeat_interleave, float mask, SDPA, and the
    host read of kv_len.max()) runs on the same inputs for comparison.  One JSON line.
    """
    import torch.nn.functional as F
    from mimir_amd.cache import Cache, attention_with_cache

    B, hq, hkv, d, L = 8, 16, 4, 128, 4096
    gen = torch.Generator().manual_seed(args.seed)
    lens = torch.randint(1024, 4096 - 512, (B,), generator=gen)
    ck = torch.randn(B, L, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
    cv = torch.randn(B, L, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
    cache = Cache(ck, cv)

    def reference(q, k, v, cache_lengths, causal):
        batch_size, seqlen = q.shape[:2]
        positions = cache_lengths[:, None] + torch.arange(seqlen, device=dev, dtype=cache_lengths.dtype)
        rows = torch.arange(batch_size, device=dev)
        cache.keys[rows[:, None], positions] = k
        cache.values[rows[:, None], positions] = v
        kv_len = cache_lengths + seqlen
        m = kv_len.max().item()
        keys = cache.keys[:batch_size, :m].repeat_interleave(hq // hkv, dim=2)
        values = cache.values[:batch_size, :m].repeat_interleave(hq // hkv, dim=2)
        kp = torch.arange(m, device=dev)
        valid = kp[None, :] < kv_len[:, None]
        valid = valid[:, None, :] & (kp[None, None, :] <= positions[:, :, None]) if causal else valid[:, None, :]
        mask = torch.zeros((batch_size, seqlen, m), dtype=q.dtype, device=dev).masked_fill(~valid, torch.finfo(q.dtype).min)
        return F.scaled_dot_product_attention(q.transpose(1, 2), keys.transpose(1, 2), values.transpose(1, 2),
                                              attn_mask=mask[:, None]).transpose(1, 2)

    def timed(fn, steps, warmup):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    K, W = max(1, args.steps), max(1, args.warmup)
    res = {"metric": "KV-cache decode attention GB/s (cache read)", "unit": "GB/s", "higher_is_better": True,
           "steps": K, "warmup": W, "dtype": "bf16", "data": "synthetic",
           "config": {"batch": B, "q_heads": hq, "kv_heads": hkv, "head_dim": d, "cache_len": L,
                      "cache_lengths": lens.tolist(), "seed": args.seed}}
    for name, S, causal in (("decode", 1, True), ("prefill", 512, True)):
        cl = (lens if name == "decode" else torch.full((B,), 1536)).to(dev)
        q = torch.randn(B, S, hq, d, generator=gen).to(torch.bfloat16).to(dev)
        k = torch.randn(B, S, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
        v = torch.randn(B, S, hkv, d, generator=gen).to(torch.bfloat16).to(dev)
        ms = timed(lambda: attention_with_cache(q, k, v, cache, cl, causal), K, W)
        ms_ref = timed(lambda: reference(q, k, v, cl, causal), K, W)
        kv = (cl.cpu() + S).tolist()
        cache_bytes = sum(kv) * hkv * d * 2 * 2
        io_bytes = 2 * B * S * hq * d * 2 + 2 * B * S * hkv * d * 2
        pairs = sum(c * S + S * (S + 1) // 2 for c in cl.cpu().tolist())  # allowed (query, key) pairs
        entry = {"ms": round(ms, 5), "reference_ms": round(ms_ref, 5), "speedup_vs_reference": round(ms_ref / ms, 2),
                 "gbs": round((cache_bytes + io_bytes) / (ms * 1e-3) / 1e9, 1),
                 "tflops": round(4 * d * hq * pairs / (ms * 1e-3) / 1e12, 2)}
        entry["hbm_frac"] = round(entry["gbs"] / HBM_GBS, 4)
        if name == "decode":
            # The same decode step captured in a HIP graph and replayed (for callers that capture
            # their decode loop; on this short two-kernel graph the replay overhead exceeds the
            # eager call's host work, so `ms` stays the reported rate).
            fn = lambda: attention_with_cache(q, k, v, cache, cl, causal)
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                fn()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                fn()
            gms = timed(graph.replay, K, W)
            entry["graph_ms"] = round(gms, 5)
            entry["graph_gbs"] = round((cache_bytes + io_bytes) / (gms * 1e-3) / 1e9, 1)
        res[name] = entry
    res["value"] = res["decode"]["gbs"]
    res["roofline"] = {"kernel": "cache_append_kernel + cache_attn_kernel<128> (decode step)", "bound": "hbm",
                       "achieved": res["decode"]["gbs"], "peak": HBM_GBS, "unit": "GB/s",
                       "frac": res["decode"]["hbm_frac"]}
    print(json.dumps(res), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-seconds", type=float, default=1.0,
                    help="warm up for at least this long (and at least --warmup steps) so that the GPU clocks settle "
                         "before anything is timed")
    ap.add_argument("--workload", type=int, default=2, choices=[1, 2, 3, 4, 5, 6])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--layer", action="store_true",
                    help="instead of the operator, time the attention layer core (gqkv split, RoPE, attention, "
                         "sigmoid gate; fwd+bwd) fused (mimir_amd.layer) against the reference's composition of "
                         "torch ops around the same operator")
    ap.add_argument("--cache", action="store_true",
                    help="instead of the operator, time KV-cache attention (inference): decode (S = 1) and a "
                         "prefill chunk into a filled cache, fused (mimir_amd.cache) against the reference's "
                         "torch composition")
    ap.add_argument("--autograd", action="store_true",
                    help="time the drop-in as Mimir2 calls it: flash_attn_varlen_prefixlm through autograd "
                         "(custom ops, argument checks, allocation of outputs and workspaces) and .backward(), "
                         "instead of replaying prepared C-ABI calls")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="instead of the step, time a plain device copy of this many MiB (reference kernel of known "
                         "HBM traffic for scaling the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): the operator runs on one GPU's "
              "share of the workload; sharding it over GPUs (documents and heads, no exchange) is not launched here.",
              file=sys.stderr)
        return 2

    import torch

    from mimir_amd import _capi
    from mimir_amd import prefixlm as P
    from mimir_amd.workloads import CONFIG_NAMES, bwd_bytes, fwd_bytes, make_config

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    if args.copy_calibration_mib > 0:
        return copy_calibration(torch, dev, args.copy_calibration_mib, max(1, args.steps))
    if args.layer:
        return layer_bench(torch, dev, args)
    if args.cache:
        return cache_bench(torch, dev, args)
    case = make_config(args.workload, seed=args.seed)
    c = case.to(dev)
    T, hq, d = c.q.shape
    hkv = c.k.shape[1]
    elem = c.q.element_size()
    scale = 1.0 / math.sqrt(d)
    lib = _capi.load()
    stream = torch.cuda.current_stream(dev).cuda_stream

    # as the autograd path runs it: for bf16 the forward records its split decision
    # (split mode AUTO) and writes the low output half when it splits; the backward
    # follows that decision and reads the low half for its delta rows then
    out_lo = torch.empty_like(c.q) if elem == 2 else None
    flag = torch.empty(1 if elem == 2 else 0, dtype=torch.int32, device=dev)
    fp, out, lse, keep_f = P.prepare_fwd(c.q, c.k, c.v, case.is_causal, c.prefix_lens, c.causal_lens, c.cu_seqlens,
                                         c.total_seqlen, c.numseqs, c.max_seqlen_all, scale, out_lo=out_lo,
                                         split_flag=flag)
    _capi.raise_for_status(lib, lib.mimir_prefixlm_fwd(ctypes.byref(fp), stream))
    bp, dq, dk, dv, keep_b = P.prepare_bwd(c.dout, c.q, c.k, c.v, out, lse, case.is_causal, c.prefix_lens,
                                           c.causal_lens, c.cu_seqlens, c.total_seqlen, c.numseqs,
                                           c.max_seqlen_all, scale, out_lo=out_lo, split_flag=flag)
    fwd_only = args.workload == 1
    stages = [("fwd", None)]
    if not fwd_only:
        stages += [("delta", _capi.BWD_STAGE_DELTA), ("dkdv", _capi.BWD_STAGE_DKDV), ("dq", _capi.BWD_STAGE_DQ),
                   ("fill", _capi.BWD_STAGE_FILL)]
    fwd_fn, stg_fn = lib.mimir_prefixlm_fwd, lib.mimir_prefixlm_bwd_stages
    fpr, bpr = ctypes.byref(fp), ctypes.byref(bp)

    bwd_fn = lib.mimir_prefixlm_bwd

    if args.autograd:
        from mimir_amd import flash_attn_varlen_prefixlm

        qg, kg, vg = (t.detach().clone().requires_grad_(not fwd_only) for t in (c.q, c.k, c.v))
        call_args = (c.prefix_lens, c.causal_lens, c.cu_seqlens, c.total_seqlen, c.numseqs, c.max_seqlen_prefix,
                     c.max_seqlen_causal, c.max_seqlen_all)

        def run_fwd():
            return flash_attn_varlen_prefixlm(qg, kg, vg, case.is_causal, *call_args)

        def run_bwd(o):
            # q / k / v stand for the views of the projection they are in Mimir2 (layers.py:183-189):
            # gradients flow on instead of accumulating into leaves, so no grad accumulation kernels
            qg.grad = kg.grad = vg.grad = None
            o.backward(c.dout)

        def step():
            """flash_attn_varlen_prefixlm + .backward(): host checks, allocations and launches included."""
            o = run_fwd()
            if not fwd_only:
                run_bwd(o)
    else:
        def run_fwd():
            rc = fwd_fn(fpr, stream)
            if rc:
                _capi.raise_for_status(lib, rc)

        def run_bwd(_):
            rc = bwd_fn(bpr, stream)
            if rc:
                _capi.raise_for_status(lib, rc)

        def step():
            """One operator step as the autograd path runs it: forward, then the whole backward."""
            o = run_fwd()
            if not fwd_only:
                run_bwd(o)

    def staged_step(evs):
        """The same work one stage at a time, with HIP events between the stages."""
        for i, (name, bits) in enumerate(stages):
            evs[i].record()
            rc = fwd_fn(fpr, stream) if bits is None else stg_fn(bpr, bits, stream)
            if rc:
                _capi.raise_for_status(lib, rc)
        evs[len(stages)].record()

    K = args.steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(stages) + 1)] for _ in range(K)]
    # Warm-up by time: at least --warmup steps and at least --warmup-seconds of them
    # (each step synchronized, so the host clock measures GPU work), so that the
    # clocks have settled before the timed region.
    t_warm = time.perf_counter()
    warm_steps = 0
    while warm_steps < args.warmup or time.perf_counter() - t_warm < args.warmup_seconds:
        step()
        torch.cuda.synchronize()
        warm_steps += 1
    warm_s = time.perf_counter() - t_warm

    # Timed region (the `value`): K whole steps back to back, one event before the
    # first and one after the last.
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for _ in range(K):
        step()
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / K

    # The same K steps again with an event at every step boundary: per-step
    # durations (their median, and their mean for comparison with the timed region).
    be = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    be[0].record()
    for k in range(K):
        step()
        be[k + 1].record()
    torch.cuda.synchronize()
    per_step = [be[k].elapsed_time(be[k + 1]) for k in range(K)]
    step_med = statistics.median(per_step)
    step_evented_mean = be[0].elapsed_time(be[K]) / K

    # Forward alone per step, events around it: median of K runs.
    pe = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(K)]
    for k in range(K):
        pe[k][0].record()
        o = run_fwd()
        pe[k][1].record()
        if not fwd_only:
            run_bwd(o)
    torch.cuda.synchronize()
    fwd_med = statistics.median(e[0].elapsed_time(e[1]) for e in pe)

    # Per-kernel durations: K more steps with the stages serialized and bracketed by events.
    for k in range(K):
        staged_step(evs[k])
    torch.cuda.synchronize()

    stage_ms = {name: [evs[k][i].elapsed_time(evs[k][i + 1]) for k in range(K)] for i, (name, _) in enumerate(stages)}
    stage_avg = {name: sum(v) / len(v) for name, v in stage_ms.items()}
    stage_med = {name: statistics.median(v) for name, v in stage_ms.items()}
    staged_med = statistics.median(sum(stage_ms[n][k] for n, _ in stages) for k in range(K))

    pairs = case.pairs()
    f_fwd = 4.0 * d * hq * pairs
    f_bwd = 0.0 if fwd_only else 10.0 * d * hq * pairs
    flops = f_fwd + f_bwd
    value = flops / (ms_per_step * 1e-3) / 1e12
    peak = PEAK_F32_TFLOPS if c.q.dtype == torch.float32 else PEAK_BF16_TFLOPS
    kernel_flops = {"fwd": f_fwd, "dkdv": 8.0 * d * hq * pairs, "dq": 2.0 * d * hq * pairs}
    handoff = not fwd_only and int(lib.mimir_prefixlm_bwd_dscore_bytes(bpr)) > 0  # dQ reads dK/dV's dS
    # with the split the recomputing dQ does the work even where the hand-off region exists
    split = auto_split(case, scale)
    handoff = handoff and not split
    kernel_names = working_kernels(d, elem, handoff)
    dom = max((n for n in kernel_flops if n in stage_avg), key=lambda n: stage_avg[n])
    achieved = kernel_flops[dom] / (stage_avg[dom] * 1e-3) / 1e12
    alg_bytes = fwd_bytes(T, hq, hkv, d, elem) + (0 if fwd_only else bwd_bytes(T, hq, hkv, d, elem))

    res = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if elem == 2 else "f32",
        "data": "synthetic",
        "config": {
            "workload": CONFIG_NAMES[args.workload],
            "tokens": T, "seqs": len(case.seq_lens), "max_seq_len": max(case.seq_lens),
            "q_heads": hq, "kv_heads": hkv, "head_dim": d, "seed": args.seed,
            "attended_pairs": pairs, "passes": "fwd" if fwd_only else "fwd+bwd",
            "parallelism": "single-gpu",
            "path": ("flash_attn_varlen_prefixlm + autograd backward (host work included)" if args.autograd
                     else "C-ABI mimir_prefixlm_fwd + mimir_prefixlm_bwd, prepared parameter structs"),
        },
        "pct_of_peak": round(100.0 * value / peak, 2),
        "hbm_gbs_algorithmic": round(alg_bytes / (ms_per_step * 1e-3) / 1e9, 1),
        "timing": ("value = attended FLOPs / ms_per_step, ms_per_step = the mean of K back-to-back steps between "
                   "two events after a time-based warm-up; step_ms_median = the median of K per-step durations from a "
                   "second pass of K steps with an event at every step boundary (step_ms_evented_mean = that pass's "
                   "mean)"),
        "warmup_steps_run": warm_steps,
        "warmup_s": round(warm_s, 3),
        "fwd_ms_median": round(fwd_med, 5),
        "step_ms_median": round(step_med, 5),
        "step_ms_evented_mean": round(step_evented_mean, 5),
        "step_ms_min": round(min(per_step), 5),
        "step_ms_max": round(max(per_step), 5),
        "fwd_tflops_median": round(f_fwd / (fwd_med * 1e-3) / 1e12, 2),
        "step_tflops_median": round(flops / (step_med * 1e-3) / 1e12, 2),
        "staged_step_ms_median": round(staged_med, 5),
        "stage_ms_avg": {n: round(v, 5) for n, v in stage_avg.items()},
        "stage_ms_median": {n: round(v, 5) for n, v in stage_med.items()},
        "fwd_tflops": round(f_fwd / (stage_avg["fwd"] * 1e-3) / 1e12, 2),
        "roofline": {
            "kernel": kernel_names[dom],
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": None,
            "algorithmic_flops_per_launch": kernel_flops[dom],
        },
    }
    measured = _measured_traffic(CONFIG_NAMES[args.workload], kernel_names[dom])
    if measured is not None:
        res["roofline"]["traffic"] = measured["bytes"]
        res["roofline"]["traffic_source"] = measured["source"]
        # the same kernel's measured HBM traffic over its duration: how close it also is to the
        # HBM bound (with the dS hand-off the dK/dV kernel streams 0.7 GB of dS out)
        gbs = measured["bytes"] / (stage_avg[dom] * 1e-3) / 1e9
        res["roofline"]["traffic_gbs"] = round(gbs, 1)
        res["roofline"]["traffic_frac_of_hbm"] = round(gbs / HBM_GBS, 4)
    if not fwd_only:
        res["bwd_tflops"] = round(f_bwd / ((ms_per_step - stage_avg["fwd"]) * 1e-3) / 1e12, 2)
    res["dscore_handoff"] = handoff
    if elem == 2 and not fwd_only:
        res["split_active"] = split
    if handoff:
        # the dQ kernel is then HBM-bound: it streams every stored dS block once
        # (plus K once and the dQ rows)
        ds_bytes = dscore_blocks(case) * hq * 2048 + T * (hkv + hq) * d * elem
        res["dq_ds_bytes"] = ds_bytes
        res["dq_ds_gbs"] = round(ds_bytes / (stage_avg["dq"] * 1e-3) / 1e9, 1)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(case)
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
