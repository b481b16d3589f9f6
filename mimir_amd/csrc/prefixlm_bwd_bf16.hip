// bf16 prefix-LM attention backward for gfx950 (MI355X): an atomic-free split
// into three kernels, the same ownership split as the reference's Metal
// backward (flash_attention_prefixlm_mps.py:867-898 delta, 967-1039 dQ per query
// row, 1245-1322 dK/dV per key row), re-tiled for bf16 MFMA.
//
//   delta:  delta[h, t] = sum_d O[t, h, d] * dO[t, h, d]                 (fp32)
//   dq:     owner = (query head, 128 query rows).  Per 64-key tile:
//             S^T = K Q^T, dP^T = V dO^T, P^T = exp(scale*S^T - lse),
//             dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.
//   dkdv:   owner = (kv head, key tile).  Per q-head of the GQA group and per
//           64-query tile:  S = Q K^T, dP = dO V^T, P, dS as above,
//             dV^T += dO^T P,  dK^T += Q^T dS.
//           The GQA reduction over the q-heads of one kv head happens in
//           registers, so no kernel needs atomics and results are deterministic.
//
// This file holds the delta kernel and the orchestration; the dQ and dK/dV
// kernels live in prefixlm_bwd_dq_bf16.hip and prefixlm_bwd_dkdv_bf16.hip.  Both
// tile loops stream their operand tiles with direct buffer-to-LDS loads into two
// LDS stages (one barrier per tile).  Grids are ordered so that the heaviest
// tiles of every sequence are dispatched first.
//
// Math: dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta) * scale,
// dQ = dS K, dK = dS^T Q  (flash_attention_prefixlm_mps.py:1601-1675), with the GQA
// head map of flash_attention_prefixlm_dense.py:10-16 (q head h -> kv head h / G).
#include "prefixlm_bwd_bf16.h"

namespace {
using namespace mimir;

// ---------------------------------------------------------------------------
// delta = rowsum(O * dO), one (token, head) row per D/8 lanes; the same pass
// stores lse * log2(e), so the tile loops form P = exp2(S * scale * log2(e) - lse2)
// with one FMA per score.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void delta_kernel(const BwdArgs a) {
  constexpr int LPR = D / 8;  // lanes per row
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / LPR;  // row = t * Hq + h
  const int c = (int)(gid % LPR);
  const bool valid = row < (int64_t)a.T * a.Hq;
  const int t = valid ? (int)(row / a.Hq) : 0;
  const int h = valid ? (int)(row % a.Hq) : 0;
  float acc = 0.f;
  if (valid) {
    const bf16x8 ov = *(const bf16x8*)&a.o[(int64_t)t * a.o_st + (int64_t)h * a.o_sh + c * 8];
    const bf16x8 dv = *(const bf16x8*)&a.dout[(int64_t)t * a.do_st + (int64_t)h * a.do_sh + c * 8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (float)ov[e] * (float)dv[e];
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (valid && c == 0) {
    a.delta[(int64_t)h * a.T + t] = acc;
    a.lse2[(int64_t)h * a.T + t] = a.lse[(int64_t)h * a.lse_sh + t] * kLog2e;
  }
}

template <int D>
hipError_t launch(const MimirPrefixLMBwdParams& p, hipStream_t stream, int stages) {
  BwdArgs a;
  a.q = (const bf16_t*)p.q;
  a.k = (const bf16_t*)p.k;
  a.v = (const bf16_t*)p.v;
  a.o = (const bf16_t*)p.out;
  a.dout = (const bf16_t*)p.dout;
  a.lse = p.lse;
  a.dq = (bf16_t*)p.dq;
  a.dk = (bf16_t*)p.dk;
  a.dv = (bf16_t*)p.dv;
  a.delta = (float*)p.workspace;
  a.lse2 = (float*)p.workspace + (int64_t)p.num_q_heads * p.total_tokens;
  a.plan_cap = plan_capacity(p.total_tokens, p.numseqs, p.max_seqlen_all);
  a.plan_q = (int2*)((float*)p.workspace + 2 * (int64_t)p.num_q_heads * p.total_tokens);
  a.plan_k = a.plan_q + a.plan_cap;
  a.plan = nullptr;
  a.prefix_lens = p.prefix_lens;
  a.cu_seqlens = p.cu_seqlens;
  a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.k_st = p.k_stride_token; a.k_sh = p.k_stride_head;
  a.v_st = p.v_stride_token; a.v_sh = p.v_stride_head;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.do_st = p.dout_stride_token; a.do_sh = p.dout_stride_head;
  a.dq_st = p.dq_stride_token; a.dq_sh = p.dq_stride_head;
  a.dk_st = p.dk_stride_token; a.dk_sh = p.dk_stride_head;
  a.dv_st = p.dv_stride_token; a.dv_sh = p.dv_stride_head;
  a.lse_sh = p.lse_stride_head;
  a.T = p.total_tokens;
  a.Hq = p.num_q_heads;
  a.Hkv = p.num_kv_heads;
  a.group = p.num_q_heads / p.num_kv_heads;
  a.total_seqlen = p.total_seqlen;
  a.is_causal = p.is_causal;
  a.scale = p.softmax_scale;
  a.scale_log2 = p.softmax_scale * kLog2e;

  const int64_t rows = (int64_t)p.total_tokens * p.num_q_heads;
  if (rows > 0 && (stages & MIMIR_BWD_STAGE_DELTA)) {
    const int64_t threads = rows * (D / 8);
    hipLaunchKernelGGL(delta_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (stages & MIMIR_BWD_STAGE_DKDV) {
    e = D == 128 ? launch_bwd_dkdv_pair_bf16(a, p.numseqs, p.max_seqlen_all, stream)
                 : launch_bwd_dkdv_bf16(a, D, p.numseqs, p.max_seqlen_all, stream);
    if (e != hipSuccess) return e;
  }
  if (stages & MIMIR_BWD_STAGE_DQ) {
    e = launch_bwd_dq_bf16(a, D, p.numseqs, p.max_seqlen_all, stream);
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t mimir_launch_bwd_bf16(const MimirPrefixLMBwdParams& p, hipStream_t stream, int stages) {
  switch (p.head_dim) {
    case 64: return launch<64>(p, stream, stages);
    case 128: return launch<128>(p, stream, stages);
    default: return hipErrorInvalidValue;
  }
}
