// bf16 prefix-LM attention backward for gfx950 (MI355X): an atomic-free split
// into three kernels, the same ownership split as the reference's Metal
// backward (flash_attention_prefixlm_mps.py:867-898 delta, 967-1039 dQ per query
// row, 1245-1322 dK/dV per key row), re-tiled for bf16 MFMA.
//
//   delta:  delta[h, t] = sum_d O[t, h, d] * dO[t, h, d]                 (fp32)
//   dq:     owner = (query head, 128 query rows).  Per 64-key tile:
//             S^T = K Q^T, dP^T = V dO^T, P^T = exp(scale*S^T - lse),
//             dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.
//           With the score-gradient hand-off (head_dim 128) the dK/dV kernel
//           stores its bf16 dS tiles and dQ^T += K^T dS^T reads them instead.
//   dkdv:   owner = (kv head, key tile).  Per q-head of the GQA group and per
//           64-query tile:  S = Q K^T, dP = dO V^T, P, dS as above,
//             dV^T += dO^T P,  dK^T += Q^T dS.
//           The GQA reduction over the q-heads of one kv head happens in
//           registers, so no kernel needs atomics and results are deterministic.
//
// This file holds the orchestration.  The delta rows (with lse * log2(e)) and
// both tile work lists come from the prologue launch (prefixlm_prologue.hip) of
// the DELTA stage; the dQ kernel lives in prefixlm_bwd_dq_bf16.hip, the dK/dV
// kernels in prefixlm_bwd_dkdv_pair_bf16.hip (head_dim 128) and
// prefixlm_bwd_dkdv_bf16.hip (head_dim 64).  The tile loops stream their operand
// tiles with direct buffer-to-LDS loads into multi-stage LDS rings, and every
// workgroup takes its tile from a heaviest-first work list.
//
// Math: dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta) * scale,
// dQ = dS K, dK = dS^T Q  (flash_attention_prefixlm_mps.py:1601-1675), with the GQA
// head map of flash_attention_prefixlm_dense.py:10-16 (q head h -> kv head h / G).
#include "prefixlm_bwd_bf16.h"

namespace {
using namespace mimir;

template <int D>
hipError_t launch(const MimirPrefixLMBwdParams& p, Prologue pro, hipStream_t stream, int stages) {
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
  const bool gated = p.gate != nullptr;
  const size_t ds_bytes = mimir_prefixlm_bwd_dscore_bytes(&p);
  const BwdWorkspace ws = bwd_workspace_layout(p.total_tokens, p.num_q_heads, p.numseqs, p.max_seqlen_all,
                                               gated ? (size_t)p.total_tokens * p.num_q_heads * D * 2 : 0, ds_bytes,
                                               bwd_chunk_head_dim(p));
  char* const wsb = (char*)p.workspace;
  const DscoreGeom dsg = dscore_geometry(p.total_tokens, p.num_q_heads, p.numseqs, p.max_seqlen_all);
  a.dscore = ds_bytes > 0 ? (bf16_t*)(wsb + ws.dscore) : nullptr;
  a.ds_rows = dsg.rows;
  a.ds_width = dsg.width;
  a.delta = (float*)(wsb + ws.delta);
  a.lse2 = (float*)(wsb + ws.lse2);
  // with key-range chunks the dQ list lives in the chunk section, with room for the parts
  a.plan_q = (int4*)(wsb + (ws.chunk_slots > 0 ? ws.chunk_list : ws.plan_q));
  a.plan_k = (int4*)(wsb + ws.plan_k);
  a.cap_q = ws.cap_q + ws.chunk_slots;
  a.chunk_ctr = ws.chunk_slots > 0 ? (int*)(wsb + ws.chunk_ctr) : nullptr;
  a.chunk_part = ws.chunk_slots > 0 ? wsb + ws.chunk_part : nullptr;
  a.cap_k = ws.cap_k;
  a.plan = a.plan_q;
  a.split_ctr = (int*)(wsb + ws.counters);
  a.queue = a.split_ctr + ws.pair_heads;
  a.split_buf = (float*)(wsb + ws.slots);
  a.prefix_lens = p.prefix_lens;
  a.cu_seqlens = p.cu_seqlens;
  a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.k_st = p.k_stride_token; a.k_sh = p.k_stride_head;
  a.v_st = p.v_stride_token; a.v_sh = p.v_stride_head;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.do_st = p.dout_stride_token; a.do_sh = p.dout_stride_head;
  if (gated) {  // the tile kernels read the upstream gradient the DELTA stage forms in the workspace
    a.dout = (const bf16_t*)(wsb + ws.dout);
    a.do_st = (int64_t)p.num_q_heads * D;
    a.do_sh = D;
  }
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
  a.kscan = (const int*)(wsb + ws.kscan);
  a.split_flag = p.split_flag;
  a.split_mode = p.split_mode;
  a.rope = RopeTab{p.rope_cos, p.rope_sin, p.rope_stride_token};

  if (stages & MIMIR_BWD_STAGE_DELTA) {
    DeltaArgs& d = pro.delta;
    d.o = a.o; d.dout = (const bf16_t*)p.dout; d.lse = a.lse; d.delta = a.delta; d.lse2 = a.lse2;
    d.o_lo = (const bf16_t*)p.out_lo;
    d.lo_gate = p.split_flag;
    d.olo_st = p.out_lo_stride_token; d.olo_sh = p.out_lo_stride_head;
    d.o_st = a.o_st; d.o_sh = a.o_sh; d.do_st = p.dout_stride_token; d.do_sh = p.dout_stride_head;
    d.lse_sh = a.lse_sh;
    d.T = a.T; d.Hq = a.Hq; d.D = D;
    d.gate = gated ? (const bf16_t*)p.gate : nullptr;
    d.dgate = (bf16_t*)p.dgate;
    d.dout_s = (bf16_t*)a.dout;
    d.g_st = p.gate_stride_token; d.g_sh = p.gate_stride_head;
    d.dg_st = p.dgate_stride_token; d.dg_sh = p.dgate_stride_head;
    d.ds_st = a.do_st; d.ds_sh = a.do_sh;
    pro.has_delta = 1;
    // both tile lists: the dK/dV stage reads kind 1, the dQ stage kind 0
    PlanArgs pk = plan_args(p.cu_seqlens, p.prefix_lens, p.numseqs, p.total_seqlen, p.is_causal, p.total_tokens,
                            /*kind=*/1, a.group, a.cap_k, a.plan_k);
    if (D == 128 && ws.pair_heads >= a.Hkv) {  // the paired kernel (one workgroup per CU) adds split partials
      pk.split_heads = a.Hkv;
      pk.max_pairs = ws.pair_heads / a.Hkv;
      pk.slots = device_cu_count();
      // a split item's first half runs the per-CU average of steps, its second the
      // rest (equal halves left the XXS queue a tail of half-units: dK/dV 0.120 ->
      // 0.108 ms there, packed documents -1%, 8 x 2048 unchanged)
      pk.span_pct = 100;
    }
    pk.zero = a.split_ctr;  // split counters, the dK / dV work queue and the dS-incomplete flag
    pk.n_zero = ws.pair_heads + kCounterWordsAfterPairs;
    pro.plan[pro.nplan++] = pk;
    PlanArgs pq = plan_args(p.cu_seqlens, p.prefix_lens, p.numseqs, p.total_seqlen, p.is_causal, p.total_tokens,
                            /*kind=*/2, a.group, a.cap_q, a.plan_q);
    if (ws.chunk_slots > 0) {  // key-range parts on small grids
      pq.split_heads = a.Hq;
      pq.slots = kChunkWgs;
      pq.max_pairs = ws.chunk_slots;
      pq.zero = a.chunk_ctr;
      pq.n_zero = ws.chunk_slots * a.Hq;
    }
    pro.plan[pro.nplan++] = pq;
    if (p.split_mode == MIMIR_SPLIT_AUTO && p.split_flag == nullptr) {  // no recorded decision: scan K
      pro.kscan = kscan_args(a.k, a.k_st, a.k_sh, a.T, a.Hkv, D, p.softmax_scale, (int*)(wsb + ws.kscan),
                             p.cu_seqlens, p.numseqs);
      pro.has_kscan = 1;
    }
  }
  hipError_t e = launch_prologue(pro, stream);
  if (e != hipSuccess) return e;
  // dK/dV (head_dim 128) runs as one persistent workgroup per CU; dQ, launched
  // behind it on a second stream, takes over each CU as its dK/dV workgroup
  // finishes and so fills the dK/dV tail.  The join makes `stream` wait for both.
  // With the score-gradient hand-off dQ reads what dK/dV wrote: one stream, in order.
  const bool both = D == 128 && a.dscore == nullptr && (stages & MIMIR_BWD_STAGE_DKDV) &&
                    (stages & MIMIR_BWD_STAGE_DQ);
  SideStream* ss = both ? side_stream() : nullptr;
  if (ss != nullptr) {
    if ((e = hipEventRecord(ss->fork, stream)) != hipSuccess) return e;
    if ((e = hipStreamWaitEvent(ss->stream, ss->fork, 0)) != hipSuccess) return e;
    if ((e = launch_bwd_dkdv_pair_bf16(a, p.numseqs, p.max_seqlen_all, stream)) != hipSuccess) return e;
    if ((e = launch_bwd_dq_bf16(a, D, p.numseqs, p.max_seqlen_all, ss->stream)) != hipSuccess) return e;
    if ((e = hipEventRecord(ss->join, ss->stream)) != hipSuccess) return e;
    return hipStreamWaitEvent(stream, ss->join, 0);
  }
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

hipError_t mimir_launch_bwd_bf16(const MimirPrefixLMBwdParams& p, Prologue pro, hipStream_t stream, int stages) {
  switch (p.head_dim) {
    case 64: return launch<64>(p, pro, stream, stages);
    case 128: return launch<128>(p, pro, stream, stages);
    default: return hipErrorInvalidValue;
  }
}
