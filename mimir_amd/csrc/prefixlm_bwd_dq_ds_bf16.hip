// bf16 prefix-LM attention backward, dQ from the stored score gradients, for
// gfx950 (MI355X).  Owner = (query head, 128 query rows), as in
// prefixlm_bwd_dq_bf16.hip; see prefixlm_bwd_bf16.hip for the split.
#include "prefixlm_bwd_bf16.h"

namespace mimir {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBlockQ = 128;  // query rows per workgroup (32 per wave)
constexpr int kBlockK = 64;   // keys per LDS tile
constexpr int kNonTemporal = 2;  // buffer cache policy: streaming (nt); dS is read once

// ---------------------------------------------------------------------------
// dQ from the stored score gradients (head_dim 128): dQ^T += K^T dS^T with dS
// read from the blocks the dK / dV kernel wrote (dscore_geometry in
// prefixlm_common.h) instead of recomputed.  Same owner, work list and K tiles
// as dq_kernel (two K stages shared by the workgroup); per 64-key tile each
// wave copies its two 2 KiB dS blocks (32 keys x its 32 queries) into its own
// LDS region -- one region per wave, refilled as soon as the wave's MFMAs have
// consumed it, which keeps the workgroup at 52 KiB of LDS and three workgroups
// per CU streaming dS -- and reads the B operand with transposing reads.  In
// LDS the second 1 KiB half of a block (positions 16..31) sits 128 bytes
// further on, so the 32 lanes of a transposing read -- key rows
// 16 (kk & 1) + 4 hi + 0..3 (and + 8) of both halves, 128 bytes each -- hit 64
// distinct banks.  Column n of the result is the block's position n, i.e.
// query ds_query_of(n) of the wave.  Blocks wholly above the diagonal were
// never written; their loads and MFMAs are skipped.
// ---------------------------------------------------------------------------
constexpr int kDsHalfElems = kDsBlockElems / 2;      // 1 KiB: 32 key rows x 16 positions
constexpr int kDsHalfStride = kDsHalfElems + 64;     // + 128 bytes
constexpr int kDsLdsBlockElems = 2 * kDsHalfStride;  // one block in LDS
constexpr int kDsWaveElems = 2 * kDsLdsBlockElems;   // one wave's dS per 64-key tile

__global__ __launch_bounds__(kThreads, 2) void dq_ds_kernel(const BwdArgs a) {
  constexpr int D = 128;
  constexpr int DT = D / 32;
  using L = TileLayout<D>;
  static_assert(kBlockK == 2 * kDsBlock, "two dS blocks per key tile");
  __shared__ __attribute__((aligned(16))) bf16_t sK0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sK1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sS[kWaves * kDsWaveElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int rank = blockIdx.x / a.Hq;
  const int h = blockIdx.x - rank * a.Hq;
  const int4 item = a.plan[rank];
  if (item.x < 0) return;  // list padding
  const int s = item.x;
  const int qtile = item.y;
  const int part = item.z & 0xff, parts = (item.z >> 8) & 0xff, span = item.z >> 16;
  const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = qtile * kBlockQ;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;
  // The stored tiles carry no low half and may be incomplete: the recomputing
  // dQ kernel enqueued beside this one does the work then.
  if (dq_needs_recompute(a, split_on(a, lane))) return;

  const int wg_kend = max(g.p, min(m0 + kBlockQ, g.nq));
  const int nkt_all = (wg_kend + kBlockK - 1) / kBlockK;
  // key tiles [kt0, nkt) of this part: the whole range unless the list cut it, then
  // the last parts `span` tiles each and the first the rest
  const int kt0 = part == 0 ? 0 : nkt_all - (parts - part) * span;
  const int nkt = nkt_all - (parts - 1 - part) * span;
  const int qa = m0 + wave * 32;
  const bool wave_active = qa < g.nq;
  const int w_kend_max = wave_active ? max(g.p, min(qa + 32, g.nq)) : 0;

  const bf16_t* kseq = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const TileLoader<D, kWaves> ldk(a.k_st, wave, lane);
  // this wave's dS block row; reads past the row (or of a row outside the
  // workspace) return zeros
  const int row = g.start / kDsBlock + s + qa / kDsBlock;
  const bool row_ok = wave_active && row < a.ds_rows;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(
      a.dscore + ((int64_t)h * a.ds_rows + (row_ok ? row : 0)) * a.ds_width * kDsBlockElems,
      row_ok ? (uint32_t)a.ds_width * kDsBlockElems * 2 : 0u);
  const uint32_t s_voff = (uint32_t)lane * 16;

  const bf16_t* i_k = kseq + (int64_t)kt0 * kBlockK * a.k_st;
  int i_rows = g.n - kt0 * kBlockK;
  int i_kt = kt0;
  auto issue_k = [&](bf16_t* tk) {
    ldk.issue_at(i_k, rows_bytes32(i_rows, (uint32_t)a.k_st, D), tk);
    i_k += kBlockK * a.k_st;
    i_rows -= kBlockK;
  };
  // dS of key tile i_kt into this wave's own LDS region (no workgroup barrier:
  // only this wave reads it)
  auto issue_ds = [&]() {
    // the blocks this wave uses: key blocks 2 i_kt (+ 1) below w_kend_max
    const int kb = i_kt * kBlockK;
    bf16_t* const dst = sS + wave * kDsWaveElems;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      if (kb + kDsBlock * mt < w_kend_max)
#pragma unroll
        for (int c = 0; c < 2; ++c)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs, (__attribute__((address_space(3))) void*)(dst + mt * kDsLdsBlockElems + c * kDsHalfStride), 16,
              s_voff,
              (uint32_t)(2 * i_kt + mt) * (kDsBlockElems * 2) + c * 1024, 0, kNonTemporal);
    ++i_kt;
  };
  if (kt0 < nkt) {
    issue_k(sK0);
    issue_ds();
  }

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = f32x16{};
  const TileLanes<D> tl(lane);
  // transposing-read lane offset inside a block: half (lane >> 4) & 1, key row
  // 4 hi + (lane & 15) / 4, positions 4 (lane & 3) .. + 3 of the half
  const int s_tr = ((lane >> 4) & 1) * kDsHalfStride + (4 * hi + ((lane & 15) >> 2)) * 16 + 4 * (lane & 3);

  auto compute = [&](int kt, const bf16_t* sK) {
    const int kb = kt * kBlockK;
    if (!wave_active || kb >= w_kend_max) return;
    const bf16_t* const sw = sS + wave * kDsWaveElems + s_tr;
    const int nkk = kb + kDsBlock < w_kend_max ? 4 : 2;  // the second block may lie wholly above the diagonal
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk >= nkk) break;
      const bf16_t* const bp = sw + (kk >> 1) * kDsLdsBlockElems + (kk & 1) * 16 * 16;
      const bf16x8 sf = cat8(lds_read_tr16(bp), lds_read_tr16(bp + 8 * 16));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const bf16_t* kp = &sK[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
        const bf16x4 k0 = lds_read_tr16(kp);
        const bf16x4 k1 = lds_read_tr16(kp + L::kTrSecond);
        dqacc[dt] = mfma32(cat8(k0, k1), sf, dqacc[dt]);
      }
    }
  };

  // The wave's dS reads of tile kt are complete (their MFMAs consumed them)
  // before its copy of tile kt + 1 into the same region is issued.
  auto next_ds = [&](int kt) {
    if (kt + 1 >= nkt) return;
    wait_lds();
    __builtin_amdgcn_sched_barrier(0);
    issue_ds();
  };
  for (int kt = kt0; kt < nkt; kt += 2) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < nkt) issue_k(sK1);
    compute(kt, sK0);
    next_ds(kt);
    if (kt + 1 >= nkt) break;
    wait_vmem();
    __syncthreads();
    if (kt + 2 < nkt) issue_k(sK0);
    compute(kt + 1, sK1);
    next_ds(kt + 1);
  }

  // A part of a cut key range: the last part of the tile to arrive sums them.
  if (__builtin_expect(parts > 1, 0) && !dq_merge_parts<DT>(a, kernel_segment(), item, h, wave, lane, dqacc)) return;

  // Epilogue: the wave stages its 32 dQ rows in LDS (half of a K stage object,
  // free once every wave is past the tile loop), in query order, and stores
  // whole rows: kRowsPerInst rows of D * 2 contiguous bytes per instruction.
  __syncthreads();
  if (!wave_active) return;
  constexpr int kPitch = D + 8;  // elements; rows stay 16-byte aligned
  constexpr int kUnits = D / 8;  // 16-byte units per row
  constexpr int kRowsPerInst = 64 / kUnits;
  static_assert(2 * 32 * kPitch <= L::kElems, "two waves' rows fit one K stage object");
  bf16_t* const stage = (wave < 2 ? sK0 : sK1) + (wave & 1) * 32 * kPitch;
  const int srow = ds_query_of(l32);
  grad_out<DT>(dqacc, a.scale, a.rope, min(g.start + qa + srow, a.T - 1), hi, [&](int dt, int rg, bf16x4 v) {
    *(bf16x4*)&stage[srow * kPitch + 32 * dt + 8 * rg + 4 * hi] = v;
  });
  // The LDS unit runs one wave's accesses in order: the reads below see the writes above.
  __asm__ volatile("" ::: "memory");
  const int u = lane % kUnits;
  bf16_t* const dbase = a.dq + (int64_t)(g.start + qa) * a.dq_st + (int64_t)h * a.dq_sh + u * 8;
#pragma unroll
  for (int j = 0; j < 32 / kRowsPerInst; ++j) {
    const int r = j * kRowsPerInst + lane / kUnits;
    const bf16x8 v = *(const bf16x8*)&stage[r * kPitch + u * 8];
    if (qa + r < g.nq) *(bf16x8*)&dbase[(int64_t)r * a.dq_st] = v;
  }
}

}  // namespace

hipError_t launch_bwd_dq_ds_bf16(const BwdArgs& a, int numseqs, hipStream_t stream) {
  static_assert(kBlockQ == kPlanTile, "work-list tiles are the dQ query tiles");
  if (numseqs <= 0 || a.cap_q == 0) return hipSuccess;
  // workgroup r * Hq + h: list entry r, head h
  hipLaunchKernelGGL(dq_ds_kernel, dim3((unsigned)a.cap_q * (unsigned)a.Hq), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
