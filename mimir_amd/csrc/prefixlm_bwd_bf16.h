// Shared argument block and launchers of the bf16 backward kernels
// (prefixlm_bwd_bf16.hip: delta + orchestration, prefixlm_bwd_dq_bf16.hip: dQ,
// prefixlm_bwd_dkdv_bf16.hip: dK / dV).
#pragma once

#include "prefixlm_common.h"

namespace mimir {

constexpr int kBwdBlockQT = 64;  // query rows per LDS tile in dK / dV

struct BwdArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  const bf16_t* o;
  const bf16_t* dout;
  const float* lse;
  bf16_t* dq;
  bf16_t* dk;
  bf16_t* dv;
  float* delta;      // workspace [Hq, T]: rowsum(dO * O)
  float* lse2;       // workspace [Hq, T]: lse * log2(e), the exp2-domain row offset
  const int32_t* prefix_lens;
  const int32_t* cu_seqlens;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, do_st, do_sh;
  int64_t dq_st, dq_sh, dk_st, dk_sh, dv_st, dv_sh, lse_sh;
  int T;
  int Hq;
  int Hkv;
  int group;
  int total_seqlen;
  int is_causal;
  int4* plan_q;      // workspace: query-tile work list (sequence, tile, part | parts << 8 | span << 16, chunk slot), for dQ
  int4* plan_k;      // workspace: key-tile work list (read by the dK / dV stage)
  int cap_q, cap_k;  // entries of each list
  const int4* plan;  // the query-tile list, for the dQ kernel
  int* chunk_ctr;    // workspace: arrival counter per (first chunk slot of a dQ tile, q head), or NULL
  char* chunk_part;  // workspace: dQ partials per (chunk slot, q head), chunk_slot_bytes(D) each
  int* split_ctr;    // workspace: arrival counter per (pair, kv head)
  int* queue;        // workspace: [0] next unit, [1] finished workgroups (dK / dV work queue)
  float* split_buf;  // workspace: two kSplitSlotFloats slots per (pair, kv head)
  bf16_t* dscore;    // workspace: bf16 dS blocks (dscore_geometry), NULL: dQ recomputes
  int ds_rows, ds_width;
  float scale;
  float scale_log2;
  const int* kscan;  // workspace: the DELTA stage's K magnitude slots (kKScanSlots)
  const int* split_flag;  // the forward's recorded split decision, or NULL
  int split_mode;    // MimirSplitMode
  RopeTab rope;      // optional: dQ / dK stored as gradients of the unrotated q / k
};

// queue[kDsIncomplete]: set by the dK / dV kernel when a score-gradient tile fell
// outside the region (zeroed by the DELTA stage with the other counters).
constexpr int kDsIncomplete = 2;

// Whether the dK and dQ products split dS into bf16 hi + lo (wave-uniform).
__device__ __forceinline__ bool split_on(const BwdArgs& a, int lane) {
  return split_decision(a.split_mode, a.kscan, a.split_flag, lane);
}
// With the score-gradient hand-off, whether the recomputing dQ kernel does the
// work instead of the one that reads the stored tiles (which have no low half).
__device__ __forceinline__ bool dq_needs_recompute(const BwdArgs& a, bool split) {
  return split || a.queue[kDsIncomplete] != 0;
}


// Key-range parts of a dQ tile (kind-2 list entry `item`, q head h): every wave
// publishes its fp32 dQ^T fragments in the part's chunk slot with device-scope
// stores and waits for them before the barrier that precedes the arrival
// count; the last part of the tile to arrive reads every part in part order
// with device-scope loads and sums them into `acc`, so the result does not
// depend on arrival order.  Returns whether this workgroup stores dQ.  Called
// by every wave of the workgroup (it holds barriers).
template <int DT>
__device__ __forceinline__ bool dq_merge_parts(const BwdArgs& a, uint64_t seg, int4 item, int h, int wave, int lane,
                                               f32x16 (&acc)[DT]) {
  __shared__ int later;
  constexpr int kDevScope = 16;  // buffer cache policy: coherent at device scope
  const int part = item.z & 0xff, parts = (item.z >> 8) & 0xff;
  const int slot0 = item.w - part;
  const uint32_t slot_bytes = (uint32_t)chunk_slot_bytes(DT * 32);
  char* const base = kernarg_at<char*>(seg, offsetof(BwdArgs, chunk_part));
  auto slot_rsrc = [&](int sl) { return make_rsrc(base + ((size_t)sl * a.Hq + h) * slot_bytes, slot_bytes); };
  auto offset = [&](int dt, int rg) { return (uint32_t)((((wave * DT + dt) * 4 + rg) * 64 + lane) * 16); };
  {
    const __amdgpu_buffer_rsrc_t r = slot_rsrc(item.w);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 v = {acc[dt][4 * rg], acc[dt][4 * rg + 1], acc[dt][4 * rg + 2], acc[dt][4 * rg + 3]};
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r, offset(dt, rg), 0, kDevScope);
      }
  }
  __asm__ volatile("" ::: "memory");
  wait_vmem();  // the slot stores are complete
  __syncthreads();
  if (threadIdx.x == 0) {
    int* const ctr = kernarg_at<int*>(seg, offsetof(BwdArgs, chunk_ctr)) + (size_t)slot0 * a.Hq + h;
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (prev == parts - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    later = prev == parts - 1;
  }
  __syncthreads();
  if (!later) return false;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
  for (int q = 0; q < parts; ++q) {
    const __amdgpu_buffer_rsrc_t r = slot_rsrc(slot0 + q);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const f32x4 v =
            __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset(dt, rg), 0, kDevScope));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[dt][4 * rg + e] += v[e];
      }
  }
  return true;
}

// Each launcher computes its own grid from the geometry in `a` and enqueues one
// kernel on `stream`.
hipError_t launch_bwd_dq_bf16(const BwdArgs& a, int head_dim, int numseqs, int max_seqlen_all, hipStream_t stream);
// head_dim 128, dQ from the score gradients the dK / dV stage stored (prefixlm_bwd_dq_ds_bf16.hip)
hipError_t launch_bwd_dq_ds_bf16(const BwdArgs& a, int numseqs, hipStream_t stream);
// head_dim 64 (prefixlm_bwd_dkdv_bf16.hip)
hipError_t launch_bwd_dkdv_bf16(const BwdArgs& a, int head_dim, int numseqs, int max_seqlen_all,
                                hipStream_t stream);
// head_dim 128, two waves per SIMD (prefixlm_bwd_dkdv_pair_bf16.hip)
hipError_t launch_bwd_dkdv_pair_bf16(BwdArgs a, int numseqs, int max_seqlen_all, hipStream_t stream);

}  // namespace mimir
