// bf16 prefix-LM attention backward, dK / dV kernel for head_dim 128 with two
// waves per SIMD, for gfx950 (MI355X).  Owner = (kv head, 128-key tile), the
// same work list as the head_dim 64 kernel in prefixlm_bwd_dkdv_bf16.hip, and
// the same math:
//   per q head of the GQA group and 64-query tile:
//     S = Q K^T, dP = dO V^T, P = exp2(S * scale * log2 e - lse2),
//     dS = P (dP - delta), dV^T += dO^T P, dK^T += Q^T dS.
//
// Workgroup = 8 waves.  Waves w and w + 4 own the same 32 keys (key slice
// w % 4, both on SIMD w % 4) and take the two 32-query halves of every 64-query
// tile (half w / 4), so each keeps its own dK / dV partial sums over half of the
// queries; the pair's partials are added through LDS at the end.  To fit two
// waves per SIMD (256 registers each) only the K fragments stay in registers:
// the 128 x 128 V tile is staged in LDS once and read as the B operand of dP.
// With two waves per SIMD the hardware overlaps one wave's softmax with the
// other's MFMAs.
//
// dkdv_pair_ds_kernel also stores each step's bf16 dS (32 queries x the wave's
// 32 keys, one 2 KiB block, dscore_geometry in prefixlm_common.h) for the dQ
// stage, which then needs no recompute of S and dP.
#include "prefixlm_bwd_bf16.h"

namespace mimir {
namespace {

constexpr int kPairWaves = 8;
constexpr int kNonTemporal = 2;  // buffer cache policy: streaming (nt)
constexpr int kPairKeys = 128;
constexpr int kPairD = 128;

// LDS: three stages of (Q tile, dO tile, lse2 row, delta row) and the V tile
// (two 64-row TileLayout tiles).  Each stage is one object, so that the
// compiler can tell the reads of one stage from the tile copies into another (it
// tracks the copy targets of a few objects only: with one object per tile it
// made some stage's reads wait for every copy in flight).  Declared apart from
// the body, so that a kernel's plain and split bodies share them.  After the
// tile loop the Q / dO tiles of stages 0 and 1 hold the dK / dV partials of the
// second wave of each pair.
constexpr int kStageElems = 2 * TileLayout<kPairD>::kElems + 2 * kBwdBlockQT * 2;  // Q, dO, lse2 + delta (fp32)
struct PairLds {
  bf16_t *s0, *s1, *s2, *v;
  int *unit_next, *later;
};
__device__ __forceinline__ PairLds pair_lds() {
  __shared__ __attribute__((aligned(16))) bf16_t sS0[kStageElems];
  __shared__ __attribute__((aligned(16))) bf16_t sS1[kStageElems];
  __shared__ __attribute__((aligned(16))) bf16_t sS2[kStageElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV[2 * TileLayout<kPairD>::kElems];
  __shared__ int unit_next;
  __shared__ int later;
  return PairLds{sS0, sS1, sS2, sV, &unit_next, &later};
}

template <bool kStoreDs, bool kSplit>
__device__ __forceinline__ void dkdv_pair_body(const BwdArgs& a, uint64_t seg) {
  constexpr int D = kPairD;
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  using L = TileLayout<D>;
  using Loader = TileLoader<D, kPairWaves>;
  static_assert(kBwdBlockQT == 64, "one TileLayout tile per Q / dO block");

  const PairLds lds = pair_lds();
  bf16_t* const sS0 = lds.s0;
  bf16_t* const sS1 = lds.s1;
  bf16_t* const sS2 = lds.s2;
  bf16_t* const sV = lds.v;
  int& unit_next = *lds.unit_next;  // the workgroup's next work unit
  int& later = *lds.later;          // split tiles: 1 if this half arrived second
  bf16_t* const sQ0 = sS0;
  bf16_t* const sO0 = sS0 + L::kElems;
  float* const sL0 = (float*)(sS0 + 2 * L::kElems);
  float* const sD0 = sL0 + kBwdBlockQT;
  bf16_t* const sQ1 = sS1;
  bf16_t* const sO1 = sS1 + L::kElems;
  float* const sL1 = (float*)(sS1 + 2 * L::kElems);
  float* const sD1 = sL1 + kBwdBlockQT;
  bf16_t* const sQ2 = sS2;
  bf16_t* const sO2 = sS2 + L::kElems;
  float* const sL2 = (float*)(sS2 + 2 * L::kElems);
  float* const sD2 = sL2 + kBwdBlockQT;
  static_assert(64 * 64 * 4 <= L::kElems * 2, "one slice's partials fit one tile object");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int slice = wave & 3;  // 32-key slice
  const int qh = wave >> 2;    // 32-query half of each tile
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const Loader ldq(a.q_st, wave, lane), ldo(a.do_st, wave, lane), ldv(a.v_st, wave, lane);
  const TileLanes<D> tl(lane);
  const float c2 = a.scale_log2;
  // kSplit: dS as bf16 hi + lo in the dK product (the kernels pick the body by
  // the split decision).
  auto fetch_unit = [&]() {  // next work unit from the launch-wide queue
    return (int)gridDim.x + __hip_atomic_fetch_add(&a.queue[0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };

  // One work unit: kv head hk of key-tile list entry `item`.  Thread 0 fetches
  // the workgroup's next unit into `nxt` as soon as the tile loop is done, so
  // the queue hands out units in list order to whichever workgroup frees up.
  auto run_unit = [&](const int4 item, const int hk, int& nxt) {
  const int s = item.x;
  const int half = item.z & 0xff;  // 0: the whole tile; 1 / 2: its steps before / from the split
  const int split_at = item.z >> 8;  // the split step (0: the middle)
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int kb0 = item.y * kPairKeys;
  if (kb0 >= g.n) {  // the work list holds no such tile
    if (tid == 0) nxt = fetch_unit();
    return;
  }

  const int ka = kb0 + slice * 32;  // first key of this wave's slice
  const bool wave_active = ka < g.n;
  const int qs_lane = qstart_of(g.p, ka + l32);
  const int w_qs_min = qstart_of(g.p, ka);
  const int w_qs_max = qstart_of(g.p, ka + 31);
  const int q_begin = qstart_of(g.p, kb0);
  const int nqt = g.nq > q_begin ? (g.nq - q_begin + kBwdBlockQT - 1) / kBwdBlockQT : 0;
  const int n_all = nqt * a.group;
  const int s1 = split_at > 0 ? min(split_at, n_all) : n_all / 2;
  const int it_lo = half == 2 ? s1 : 0;
  const int n_iter = (half == 1 ? s1 : n_all) - it_lo;
  const int head0 = nqt > 0 ? it_lo / nqt : 0;  // first step: q head hk * G + head0, query tile tile0
  const int tile0 = it_lo - head0 * nqt;
  // dS blocks of this wave: key block ka / 32 of block row floor(start / 32) + s + query / 32.
  // A unit whose blocks do not all fit the region (a sequence longer than
  // max_seqlen_all) stores none and flags the hand-off incomplete: the
  // recomputing dQ kernel then takes over.
  const int ds_row0 = g.start / kDsBlock + s;
  bool ds_unit_ok = true;
  if constexpr (kStoreDs) {
    ds_unit_ok = (ka >> 5) < a.ds_width && (g.nq <= 0 || ds_row0 + (g.nq - 1) / kDsBlock < a.ds_rows);
    if (!ds_unit_ok && wave_active && lane == 0) a.queue[kDsIncomplete] = 1;
  }

  const bf16_t* kseq = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const bf16_t* vseq = a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh;

  // Iteration it covers q head hk * G + it / nqt and query tile it % nqt.  The
  // tile copies walk that order with running addresses (adds only), which keeps
  // the scalar work between barrier and first MFMA short.
  const uint32_t q_st32 = (uint32_t)a.q_st, o_st32 = (uint32_t)a.do_st;
  const int qh0 = hk * a.group + head0;
  const bf16_t* q_head = a.q + ((int64_t)g.start + q_begin) * a.q_st + (int64_t)qh0 * a.q_sh;
  const bf16_t* o_head = a.dout + ((int64_t)g.start + q_begin) * a.do_st + (int64_t)qh0 * a.do_sh;
  // one 4-byte row per wave: wave 0 lse2, the others delta (same data to the same place)
  const float* r_head = (wave == 0 ? a.lse2 : a.delta) + (int64_t)qh0 * a.T + g.start + q_begin;
  const bf16_t* i_q = q_head + (int64_t)tile0 * kBwdBlockQT * a.q_st;
  const bf16_t* i_o = o_head + (int64_t)tile0 * kBwdBlockQT * a.do_st;
  const float* i_r = r_head + tile0 * kBwdBlockQT;
  int i_qt = tile0, i_rows = g.nq - q_begin - tile0 * kBwdBlockQT;
  // Every step issues its copies, also past the last tile (`valid` false): those
  // copy zero bytes (their resources are empty, so no memory is read) and only
  // write zeros to a free stage.  With the copies and the barrier waits the same
  // on every step, the compiler can see that each stage's copies are complete
  // before its reads (conditional copies made it wait for all copies in flight).
  auto issue_next = [&](bool valid, bf16_t* tq, bf16_t* to, float* tl) {
    const int rows = valid ? i_rows : 0;
    ldq.issue_at(i_q, rows_bytes32(rows, q_st32, D), tq);
    ldo.issue_at(i_o, rows_bytes32(rows, o_st32, D), to);
    const __amdgpu_buffer_rsrc_t r = make_rsrc(i_r, rows > 0 ? (uint32_t)rows * 4u : 0u);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(tl + (wave == 0 ? 0 : kBwdBlockQT)),
                                             4, (uint32_t)lane * 4u, 0, 0, 0);
    if (++i_qt == nqt) {
      i_qt = 0;
      i_rows = g.nq - q_begin;
      q_head += a.q_sh;
      o_head += a.do_sh;
      r_head += a.T;
      i_q = q_head;
      i_o = o_head;
      i_r = r_head;
    } else {
      i_rows -= kBwdBlockQT;
      i_q += kBwdBlockQT * a.q_st;
      i_o += kBwdBlockQT * a.do_st;
      i_r += kBwdBlockQT;
    }
  };

  // V tile (keys kb0 .. kb0 + 127), then the first two Q / dO stages; the K
  // fragments of this wave's slice go to registers.
  ldv.issue(vseq, kb0, g.n, sV);
  ldv.issue(vseq, kb0 + 64, g.n, sV + L::kElems);
  issue_next(n_iter > 0, sQ0, sO0, sL0);
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kseq, rows_bytes(g.n, a.k_st, D));
  bf16x8 kf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int64_t key = ka + l32;
    kf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rk, (uint32_t)((key * a.k_st + 16 * ks + 8 * hi) * 2)));
  }
  issue_next(n_iter > 1, sQ1, sO1, sL1);
  // Copies per issue_next and wave: the Q and dO loaders share one assignment,
  // so a wave with the last round's instructions (wave 0) issues 2 * kPerWave + 1
  // with its lse2 / delta row, the others two fewer.  (Giving the dO tile's last
  // instruction to wave 1 instead, as the head_dim 64 kernel does, made the
  // compiler fail on the split body here.)
  constexpr int kLoadsPerIssue = 2 * Loader::kPerWave + 1;
  // Tile `it` has landed everywhere; the copies of tile it + 1 (and dS stores
  // after them) may still be in flight.
  auto sync_stage = [&]() {
    if (ldq.has_last)
      stage_barrier<kLoadsPerIssue>();
    else
      stage_barrier<kLoadsPerIssue - 2>();
  };

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = f32x16{};
    dvacc[dt] = f32x16{};
  }
  // B operand of dP: V rows of this slice
  const bf16_t* const sVs = sV + (slice >> 1) * L::kElems + tl.op_base + (slice & 1) * 32 * L::kRowElems;

  auto compute = [&](bool masked, int qr, int head, const bf16_t* sQ, const bf16_t* sdO, const float* sL,
                     const float* sD) {  // qr = first query row of this wave's half, head = q head in the group
    f32x16 sc = f32x16{}, dp = f32x16{};
    // Per-step copies of the lane offsets: recomputing the stage addresses from
    // them each step keeps one register per offset live instead of one per
    // (stage, operand) pair, which leaves the registers for reading operands ahead.
    int opb = tl.op_base + qh * 32 * L::kRowElems, trb = tl.tr_base + qh * 32 * L::kRowElems,
        lrow = 32 * qh + 4 * hi;
    __asm__ volatile("" : "+v"(opb), "+v"(trb), "+v"(lrow));
    // The LDS operand reads run two MFMA pairs ahead of their use; the
    // scheduling barriers keep the compiler from pulling them back next to the
    // MFMAs (which would leave every MFMA waiting for its own read).
    bf16x8 qa[KS], oa[KS], va[KS];
    auto rd_a = [&](int ks) {
      qa[ks] = *(const bf16x8*)&sQ[opb + ks * 16];
      oa[ks] = *(const bf16x8*)&sdO[opb + ks * 16];
      va[ks] = *(const bf16x8*)&sVs[ks * 16];
    };
    // dV / dK operand pair j (16-query step j / 4 of this wave's half, 32 columns j % 4)
    bf16x8 ot[3], qt[3];
    auto rd_tr = [&](int j) {
      const int o = trb + (j >> 2) * 16 * L::kRowElems + (j & 3) * 32;
      ot[j % 3] = cat8(lds_read_tr16(&sdO[o]), lds_read_tr16(&sdO[o + L::kTrSecond]));
      qt[j % 3] = cat8(lds_read_tr16(&sQ[o]), lds_read_tr16(&sQ[o + L::kTrSecond]));
    };
    f32x4 l4[2], d4[2];  // lse2 / delta of the rows of one 16-query step
    auto rd_ld = [&](int s2) {
#pragma unroll
      for (int rg2 = 0; rg2 < 2; ++rg2) {
        l4[rg2] = *(const f32x4*)&sL[lrow + 8 * (2 * s2 + rg2)];
        d4[rg2] = *(const f32x4*)&sD[lrow + 8 * (2 * s2 + rg2)];
      }
    };
    f32x8 tp, tds;
    auto softmax = [&](int s2, int rg2) {  // P and dS of rows 8 (2 s2 + rg2) + 4 hi + e
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * (2 * s2 + rg2) + e;
        const float pr = fast_exp2(__builtin_fmaf(sc[r], c2, -l4[rg2][e]));
        tp[4 * rg2 + e] = pr;
        tds[4 * rg2 + e] = pr * (dp[r] - d4[rg2][e]);
      }
    };

    // S / dP MFMAs, their operands read two k-steps ahead.
    rd_a(0);
    rd_a(1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 2 < KS) rd_a(ks + 2);
      sc = mfma32(qa[ks], kf[ks], sc);
      dp = mfma32(oa[ks], va[ks], dp);
    }
    rd_ld(0);
    rd_tr(0);
    rd_tr(1);
    __builtin_amdgcn_sched_barrier(0);
    // rows of sc / dp: query qr + 8*(r/4) + 4*hi + r%4 ; column: the lane's key.
    if (masked) {
      // allowed iff qs_lane <= q < nq, i.e. (unsigned)(q - qs_lane) < (unsigned)max(nq - qs_lane, 0)
      // (no query at all for a key past the last active one).  The empty volatile
      // asm keeps this a real branch, so unmasked tiles do not pay for the compares.
      __asm__ volatile("");
      const unsigned base = (unsigned)(qr + 4 * hi - qs_lane);
      const unsigned lim = (unsigned)max(g.nq - qs_lane, 0);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (base + (unsigned)(8 * (r >> 2) + (r & 3)) >= lim) sc[r] = -INFINITY;
    }
    bf16x8 pb[2], db[2], dl[kSplit ? 2 : 1];
    // dS half s2 (positions 16 s2 .. + 15 of the block: 1 KiB of 32 key rows
    // of 32 bytes) to key row l32, positions 16 s2 + 8 hi + 0..7: one store
    // instruction writes 1 KiB contiguously, non-temporal (cache policy nt):
    // nothing reads the blocks again before the dQ kernel.  The stores join the
    // vmcnt queue behind the tile copies in flight, so the stage waits stay
    // conservative.
    __amdgpu_buffer_rsrc_t rds;
    if constexpr (kStoreDs) {
      const int row = ds_row0 + (qr >> 5);
      // region geometry loaded per step: no scalar registers held across the loop
      const int64_t blk = ((int64_t)(hk * a.group + head) * kernarg_at<int>(seg, offsetof(BwdArgs, ds_rows)) + row) *
                              kernarg_at<int>(seg, offsetof(BwdArgs, ds_width)) +
                          (ka >> 5);
      rds = make_rsrc(kernarg_at<bf16_t*>(seg, offsetof(BwdArgs, dscore)) + blk * kDsBlockElems,
                      ds_unit_ok ? kDsBlockElems * 2 : 0);
    }
    auto store_ds = [&](int s2) {
      if constexpr (kStoreDs)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, db[s2]), rds,
                                               (uint32_t)(s2 * 1024 + l32 * 32 + hi * 16), 0, kNonTemporal);
    };
    softmax(0, 0);
    softmax(0, 1);
    pb[0] = to_bf16x8(tp);
    db[0] = to_bf16x8(tds);
    if constexpr (kSplit) dl[0] = lo_half(tds, db[0]);
    store_ds(0);
    rd_ld(1);
    // Eight dV / dK MFMA pairs; the softmax of the second 16-query step runs
    // beside the first four.
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      __builtin_amdgcn_sched_barrier(0);
      if (j + 2 < 8) rd_tr(j + 2);
      const int dt = j & 3, s2 = j >> 2;
      dvacc[dt] = mfma32(ot[j % 3], pb[s2], dvacc[dt]);
      dkacc[dt] = mfma32(qt[j % 3], db[s2], dkacc[dt]);
      if constexpr (kSplit) dkacc[dt] = mfma32(qt[j % 3], dl[s2], dkacc[dt]);
      if (j == 1) softmax(1, 0);
      if (j == 2) softmax(1, 1);
      if (j == 3) {
        pb[1] = to_bf16x8(tp);
        db[1] = to_bf16x8(tds);
        if constexpr (kSplit) dl[1] = lo_half(tds, db[1]);
        store_ds(1);
      }
    }
  };
  int s_qt = tile0, s_head = head0;  // query tile and q head of the next step
  auto step = [&](const bf16_t* sQ, const bf16_t* sdO, const float* sL, const float* sD) {
    const int qr = q_begin + s_qt * kBwdBlockQT + 32 * qh;
    const int head = s_head;
    if (++s_qt == nqt) {
      s_qt = 0;
      ++s_head;
    }
    if (!wave_active || qr + 32 <= w_qs_min || qr >= g.nq) return;
    compute(qr < w_qs_max || qr + 32 > g.nq, qr, head, sQ, sdO, sL, sD);
  };

  // After the barrier of iteration it every wave is done with iteration it - 1,
  // whose stage ((it + 2) % 3) then receives tile it + 2.
  for (int it = 0; it < n_iter; it += 3) {
    sync_stage();
    issue_next(it + 2 < n_iter, sQ2, sO2, sL2);
    step(sQ0, sO0, sL0, sD0);
    if (it + 1 >= n_iter) break;
    sync_stage();
    issue_next(it + 3 < n_iter, sQ0, sO0, sL0);
    step(sQ1, sO1, sL1, sD1);
    if (it + 2 >= n_iter) break;
    sync_stage();
    issue_next(it + 4 < n_iter, sQ1, sO1, sL1);
    step(sQ2, sO2, sL2, sD2);
  }
  // The copies past the last tile, and with n_iter == 0 the V / K loads, are
  // still in flight here.
  wait_vmem();
  if (tid == 0) nxt = fetch_unit();

  // The tile buffers are free after the loop: eight 16 KiB blocks for the
  // reductions and the store transposition below.
  auto blk = [&](int i) -> bf16_t* {
    return i == 0 ? sQ0 : i == 1 ? sO0 : i == 2 ? sQ1 : i == 3 ? sO1 : i == 4 ? sQ2 : i == 5 ? sO2
         : i == 6 ? sV : sV + L::kElems;
  };
  static_assert(L::kElems * 2 >= DT * 4 * 64 * 16, "a key slice's dK or dV (fp32) fits one block");

  // Pair reduction: the second wave of each pair hands its dK and dV partials
  // over through LDS in one round (float4 per lane, lane-major: conflict-free).
  __syncthreads();  // every wave is done with the stage buffers
  {
    f32x4* const pk = (f32x4*)blk(slice) + lane;
    f32x4* const pv = (f32x4*)blk(4 + slice) + lane;
    if (qh == 1) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          pk[(dt * 4 + rq) * 64] = f32x4{dkacc[dt][4 * rq], dkacc[dt][4 * rq + 1], dkacc[dt][4 * rq + 2],
                                         dkacc[dt][4 * rq + 3]};
          pv[(dt * 4 + rq) * 64] = f32x4{dvacc[dt][4 * rq], dvacc[dt][4 * rq + 1], dvacc[dt][4 * rq + 2],
                                         dvacc[dt][4 * rq + 3]};
        }
    }
    __syncthreads();
    if (qh == 0) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 k4 = pk[(dt * 4 + rq) * 64], v4 = pv[(dt * 4 + rq) * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dkacc[dt][4 * rq + e] += k4[e];
            dvacc[dt][4 * rq + e] += v4[e];
          }
        }
    }
  }

  if (half != 0) {
    // Split tile: each half publishes its partial sums in its own slot; the
    // later of the two (per kv head) adds the other's and stores dK / dV.
    // fp32 addition commutes, so the result does not depend on which is later.
    // Slot layout: dK then dV, each four 16 KiB key-slice blocks of float4
    // (dt * 4 + rq) * 64 + lane holding acc[dt][4 rq .. 4 rq + 3].
    //
    // Visibility without cache flushes: the slot is written by device-scope
    // (write-through) stores, each wave waits for them to complete before the
    // barrier that precedes the arrival count, and the later half reads the
    // other slot with device-scope loads issued after the count has returned.
    // The loads go straight to LDS (the dead tile buffers), so all 128 KiB are
    // in flight at once.  A device-scope release / acquire fence pair would
    // instead write back and invalidate the whole L2 of the XCD, which costs the
    // other workgroups their cached Q / dO tiles.
    constexpr int kDevScope = 16;  // buffer cache policy: coherent at device scope
    constexpr uint32_t kSliceBytes = DT * 4 * 64 * 16;
    const int ph = item.w * a.Hkv + hk;
    float* const split_buf = kernarg_at<float*>(seg, offsetof(BwdArgs, split_buf));
    int* const split_ctr = kernarg_at<int*>(seg, offsetof(BwdArgs, split_ctr));
    const float* const slot_mine = split_buf + ((size_t)ph * 2 + (half - 1)) * kSplitSlotFloats;
    const float* const slot_other = split_buf + ((size_t)ph * 2 + (2 - half)) * kSplitSlotFloats;
    if (qh == 0) {
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(slot_mine, kSplitSlotFloats * 4);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const uint32_t off = slice * kSliceBytes + (uint32_t)(((dt * 4 + rq) * 64 + lane) * 16);
          const f32x4 k4 = {dkacc[dt][4 * rq], dkacc[dt][4 * rq + 1], dkacc[dt][4 * rq + 2], dkacc[dt][4 * rq + 3]};
          const f32x4 v4 = {dvacc[dt][4 * rq], dvacc[dt][4 * rq + 1], dvacc[dt][4 * rq + 2], dvacc[dt][4 * rq + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, k4), rs, off, 0, kDevScope);
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v4), rs, off + 4 * kSliceBytes, 0,
                                                 kDevScope);
        }
      __asm__ volatile("" ::: "memory");
      wait_vmem();  // the slot stores are complete
    }
    __syncthreads();
    if (tid == 0) {
      const int prev = __hip_atomic_fetch_add(&split_ctr[ph], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (prev == 1) __hip_atomic_store(&split_ctr[ph], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      later = prev;
    }
    __syncthreads();
    if (later == 0) return;  // the other half stores the tile
    // Wave w copies block w of the other slot (dK slices 0-3, then dV) into LDS.
    {
      const __amdgpu_buffer_rsrc_t ro = make_rsrc(slot_other, kSplitSlotFloats * 4);
      bf16_t* const dst = blk(wave);
#pragma unroll
      for (int j = 0; j < DT * 4; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ro, (__attribute__((address_space(3))) void*)(dst + j * 512), 16,
                                                 wave * kSliceBytes + (uint32_t)((j * 64 + lane) * 16), 0, 0,
                                                 kDevScope);
    }
    stage_barrier<0>();
    if (qh == 0) {
      const f32x4* const ok = (const f32x4*)blk(slice) + lane;
      const f32x4* const ov = (const f32x4*)blk(4 + slice) + lane;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const f32x4 k4 = ok[(dt * 4 + rq) * 64], v4 = ov[(dt * 4 + rq) * 64];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            dkacc[dt][4 * rq + e] += k4[e];
            dvacc[dt][4 * rq + e] += v4[e];
          }
        }
    }
  }

  if (qh != 0 || !wave_active) return;
  const int kpos = ka + l32;
  if (kpos >= g.n) return;
  // the destinations loaded here: no scalar registers held across the tile loop
  bf16_t* krow = kernarg_at<bf16_t*>(seg, offsetof(BwdArgs, dk)) +
                 (int64_t)(g.start + kpos) * kernarg_at<int64_t>(seg, offsetof(BwdArgs, dk_st)) +
                 (int64_t)hk * kernarg_at<int64_t>(seg, offsetof(BwdArgs, dk_sh));
  bf16_t* vrow = kernarg_at<bf16_t*>(seg, offsetof(BwdArgs, dv)) +
                 (int64_t)(g.start + kpos) * kernarg_at<int64_t>(seg, offsetof(BwdArgs, dv_st)) +
                 (int64_t)hk * kernarg_at<int64_t>(seg, offsetof(BwdArgs, dv_sh));
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 tv;
#pragma unroll
      for (int e = 0; e < 4; ++e) tv[e] = dvacc[dt][4 * rg + e];
      *(bf16x4*)&vrow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tv, bf16x4);
    }
  grad_out<DT>(dkacc, kernarg_at<float>(seg, offsetof(BwdArgs, scale)), rope_at(seg, offsetof(BwdArgs, rope)),
               g.start + kpos, hi,
               [&](int dt, int rg, bf16x4 v) { *(bf16x4*)&krow[32 * dt + 8 * rg + 4 * hi] = v; });
  };

  // Persistent workgroups (one per CU): the first unit is the workgroup's own
  // index, later ones come from the queue, so the heaviest-first order of the
  // list holds across XCDs and no workgroup waits for a dispatch slot.
  const int n_units = a.cap_k * a.Hkv;
  int unit = blockIdx.x;
  for (;;) {
    const int rank = unit / a.Hkv;
    const int4 item = load_entry(a.plan_k, rank);
    if (item.x < 0) break;  // list padding: the rest of the list is padding too
    int nxt = n_units;
    run_unit(item, unit - rank * a.Hkv, nxt);
    if (tid == 0) unit_next = nxt;
    __syncthreads();
    unit = unit_next;
    __syncthreads();  // unit_next is rewritten after the next unit
    if (unit >= n_units) break;
  }
  // The last workgroup to leave resets the queue for the next launch.
  if (tid == 0 && __hip_atomic_fetch_add(&a.queue[1], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (int)gridDim.x - 1) {
    __hip_atomic_store(&a.queue[0], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&a.queue[1], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The split body in a function of its own, which both kernels call when the
// split is on: the plain body, inlined in the kernel, keeps the registers and
// code of a kernel of its own.  It reads its arguments from the kernel's
// argument segment `seg` (a reference to the kernel's by-value argument would
// make the compiler copy it to the stack for both bodies).  The hand-off
// stores unsplit dS only: with a split dQ the stored tiles are not used.
__device__ __attribute__((noinline)) void dkdv_pair_split_body(uint64_t seg) {
  seg = uniform_segment(seg);
  dkdv_pair_body<false, true>(segment_args<BwdArgs>(seg), seg);
}
// One launch for every split mode: the decision (the forward's recorded one, or
// the K scan's) picks the body.  Two waves per SIMD, pinned as the least and
// the most so that the called body is scheduled for that occupancy too.
#define MIMIR_PAIR_LAUNCH \
  __attribute__((amdgpu_flat_work_group_size(kPairWaves * 64, kPairWaves * 64), amdgpu_waves_per_eu(2, 2)))
__global__ MIMIR_PAIR_LAUNCH void dkdv_pair_kernel(const BwdArgs a) {
  if (split_on(a, threadIdx.x & 63))
    dkdv_pair_split_body(kernel_segment());
  else
    dkdv_pair_body<false, false>(a, kernel_segment());
}
__global__ MIMIR_PAIR_LAUNCH void dkdv_pair_ds_kernel(const BwdArgs a) {
  if (split_on(a, threadIdx.x & 63))
    dkdv_pair_split_body(kernel_segment());
  else
    dkdv_pair_body<true, false>(a, kernel_segment());
}

}  // namespace

hipError_t launch_bwd_dkdv_pair_bf16(BwdArgs a, int numseqs, int max_seqlen_all, hipStream_t stream) {
  static_assert(kPairKeys == kPlanTile, "work-list tiles are the dK / dV key tiles");
  static_assert(kPairKeys * kPairD * 2 == kSplitSlotFloats, "split slot = dK + dV of one key tile");
  if (numseqs <= 0 || a.cap_k == 0) return hipSuccess;
  // unit r * Hkv + h: list entry r (written by the DELTA stage's prologue), kv head h;
  // one persistent workgroup per CU
  const int64_t units = (int64_t)a.cap_k * a.Hkv;
  const int grid = (int)(units < device_cu_count() ? units : device_cu_count());
  hipLaunchKernelGGL(a.dscore != nullptr ? dkdv_pair_ds_kernel : dkdv_pair_kernel, dim3((unsigned)grid),
                     dim3(kPairWaves * 64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
