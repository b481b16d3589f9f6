// bf16 prefix-LM attention backward, dK / dV kernel for head_dim 64, for gfx950
// (MI355X); head_dim 128 uses prefixlm_bwd_dkdv_pair_bf16.hip.  Owner = (kv
// head, key tile); see prefixlm_bwd_bf16.hip for the split.
#include "prefixlm_bwd_bf16.h"

namespace mimir {
namespace {

// ---------------------------------------------------------------------------
// dK / dV.  Each wave owns 32 keys whose K and V fragments stay in registers as
// B operands; lanes own key columns, so P and dS feed the B operand of
// dV^T += dO^T P and dK^T += Q^T dS directly, and the transposed dO^T / Q^T
// fragments come from the row-major LDS tiles via ds_read_b64_tr_b16.
// The query range starts at qstart(first key) = (key < p ? 0 : key).
// Workgroup r * Hkv + h takes kv head h of entry r of the key-tile work list
// (prefixlm_prologue.hip): the heaviest key tiles first.
//
// Two workgroups per CU (two waves per SIMD); every operand fragment is read
// one phase ahead of its MFMAs (see compute below).
// ---------------------------------------------------------------------------
template <int D>
struct DkCfg {
  static_assert(D == 64, "head_dim 128 uses the pair kernel");
  static constexpr int kWaves = 4;                    // waves per workgroup, 32 keys each
  static constexpr int kKeys = 32 * kWaves;           // keys per workgroup
  static constexpr int kWavesPerSimd = 2;
};

// Three LDS stages of (Q tile, dO tile, lse2 row, delta row), each one object,
// so that the compiler can tell the reads of one stage from the tile copies into
// another (it tracks the copy targets of a few objects only).  Declared apart
// from the body, so that the kernel's plain and split bodies share them.
struct DkStages {
  bf16_t *s0, *s1, *s2;
};
template <int D>
__device__ __forceinline__ DkStages dk_stages() {
  constexpr int kStageElems = 2 * TileLayout<D>::kElems + 2 * kBwdBlockQT * 2;  // Q, dO, lse2 + delta (fp32)
  __shared__ __attribute__((aligned(16))) bf16_t sS0[kStageElems];
  __shared__ __attribute__((aligned(16))) bf16_t sS1[kStageElems];
  __shared__ __attribute__((aligned(16))) bf16_t sS2[kStageElems];
  return DkStages{sS0, sS1, sS2};
}

// kSplit: dS as bf16 hi + lo in the dK product (a compile-time choice: it changes
// the registers of the tile loop; the kernel below calls the split body as a
// function of its own).
template <int D, bool kSplit>
__device__ __forceinline__ void dkdv_body(const BwdArgs& a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  constexpr int kDkWaves = DkCfg<D>::kWaves;
  constexpr int kDkKeys = DkCfg<D>::kKeys;
  using L = TileLayout<D>;
  static_assert(kBwdBlockQT == 64, "one TileLayout tile per Q / dO block");
  const DkStages st = dk_stages<D>();
  bf16_t* const sS0 = st.s0;
  bf16_t* const sS1 = st.s1;
  bf16_t* const sS2 = st.s2;
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

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int rank = blockIdx.x / a.Hkv;
  const int hk = blockIdx.x - rank * a.Hkv;
  const int4 item = load_entry(a.plan_k, rank);  // never split for this kernel: part 0
  if (item.x < 0) return;  // list padding
  const int s = item.x;
  const int ktile = item.y;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int kb0 = ktile * kDkKeys;
  if (kb0 >= g.n) return;

  const int ka = kb0 + wave * 32;            // this wave's first key
  const bool wave_active = ka < g.n;
  const int qs_lane = qstart_of(g.p, ka + l32);  // first query attending this lane's key
  const int w_qs_min = qstart_of(g.p, ka);
  const int w_qs_max = qstart_of(g.p, ka + 31);
  const int q_begin = qstart_of(g.p, kb0);
  const int nqt = g.nq > q_begin ? (g.nq - q_begin + kBwdBlockQT - 1) / kBwdBlockQT : 0;
  const int n_iter = nqt * a.group;  // (q head, query tile) pairs

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(
      a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh, rows_bytes(g.n, a.k_st, D));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(
      a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh, rows_bytes(g.n, a.v_st, D));

  // Iteration it covers q head hk * G + it / nqt and query tile it % nqt.  The
  // tile copies walk that order with running addresses (adds only, no division
  // per tile).
  // Every wave issues the same number of copies per tile: the Q tile's last
  // instruction is wave 0's, the dO tile's wave 1's (rotated loader), and the
  // other waves load the lse2 row (wave 2) and the delta row (the rest).
  using Loader = TileLoader<D, kDkWaves>;
  static_assert(Loader::kInst == (Loader::kPerWave - 1) * kDkWaves + 1 && kDkWaves >= 4,
                "one last-round copy per tile, on waves 0 / 1; rows on waves 2 and up");
  const Loader ldq(a.q_st, wave, lane), ldo(a.do_st, wave, lane, 1);
  const uint32_t q_st32 = (uint32_t)a.q_st, o_st32 = (uint32_t)a.do_st;
  const int qh0 = hk * a.group;
  const bf16_t* q_head = a.q + ((int64_t)g.start + q_begin) * a.q_st + (int64_t)qh0 * a.q_sh;
  const bf16_t* o_head = a.dout + ((int64_t)g.start + q_begin) * a.do_st + (int64_t)qh0 * a.do_sh;
  // one 4-byte row per wave from wave 2 on: wave 2 lse2, the others delta (same data to the same place)
  const float* r_head = (wave == 2 ? a.lse2 : a.delta) + (int64_t)qh0 * a.T + g.start + q_begin;
  const bf16_t* i_q = q_head;
  const bf16_t* i_o = o_head;
  const float* i_r = r_head;
  int i_qt = 0, i_rows = g.nq - q_begin;
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
    if (wave >= 2)  // waves 0 / 1 issue the tiles' last copy instead
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(tl + (wave == 2 ? 0 : kBwdBlockQT)),
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
  // Three LDS stages: iteration it computes on stage it % 3 while the tiles of
  // it + 1 and it + 2 are in flight.
  issue_next(n_iter > 0, sQ0, sO0, sL0);

  bf16x8 kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int64_t key = ka + l32;
    kf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rk, (uint32_t)((key * a.k_st + 16 * ks + 8 * hi) * 2)));
    vf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rv, (uint32_t)((key * a.v_st + 16 * ks + 8 * hi) * 2)));
  }
  issue_next(n_iter > 1, sQ1, sO1, sL1);
  // Buffer loads per issue() and wave: 2 * kPerWave - 1 on every wave (Q and dO
  // tiles with the last copy of one of them, or both without it and a row).
  constexpr int kLoadsPerIssue = 2 * Loader::kPerWave - 1;
  // Tile `it` has landed everywhere; the copies of tile it + 1 may still be in flight.
  auto sync_stage = [&]() { stage_barrier<kLoadsPerIssue>(); };

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = f32x16{};
    dvacc[dt] = f32x16{};
  }
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  // One (q head, 64-query tile) step, per 32-query half h:
  //   S/dP MFMAs(h)      while the dO^T / Q^T fragments of h are read
  //   softmax(h)         (VALU)
  //   dV/dK MFMAs(h)     while the Q / dO fragments of h+1 are read
  // so every LDS fragment is read one phase before the MFMAs that use it.
  // Masked tiles (queries before some key's qstart, or past the sequence end)
  // overwrite the disallowed scores with -inf in one guarded pass right after
  // the S MFMAs.
  auto compute = [&](bool masked, int qb, const bf16_t* sQ, const bf16_t* sdO, const float* sL,
                     const float* sD) {
    bf16x8 qa[KS], da[KS];          // Q / dO rows of one half: A operands of S / dP
    bf16x8 ot[2][DT], qt[2][DT];    // dO^T / Q^T of one half: A operands of dV^T / dK^T
    auto load_s = [&](int mt) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int o = tl.op_base + mt * 32 * L::kRowElems + ks * 16;
        qa[ks] = *(const bf16x8*)&sQ[o];
        da[ks] = *(const bf16x8*)&sdO[o];
      }
    };
    auto load_t = [&](int mt) {
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int o = tl.tr_base + (2 * mt + s2) * 16 * L::kRowElems + dt * 32;
          ot[s2][dt] = cat8(lds_read_tr16(&sdO[o]), lds_read_tr16(&sdO[o + L::kTrSecond]));
          qt[s2][dt] = cat8(lds_read_tr16(&sQ[o]), lds_read_tr16(&sQ[o + L::kTrSecond]));
        }
    };

    load_s(0);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {  // 32-query halves of the tile
      f32x16 sc = f32x16{}, dp = f32x16{};
      __builtin_amdgcn_sched_barrier(0);
      load_t(mt);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        sc = mfma32(qa[ks], kf[ks], sc);
        dp = mfma32(da[ks], vf[ks], dp);
      }
      __builtin_amdgcn_sched_barrier(0);
      // rows of sc / dp: query 32*mt + 8*(r/4) + 4*hi + r%4 ; column: the lane's key.
      if (masked) {
        // allowed iff qs_lane <= q < nq, i.e. (unsigned)(q - qs_lane) < (unsigned)max(nq - qs_lane, 0):
        // a key past the last active query (nq < qs_lane, total_seqlen ending inside
        // the sequence) has no allowed query at all.  The empty volatile asm keeps
        // this block a real branch: if-converted, its 48 VALU operations would run on
        // every unmasked tile as well.
        __asm__ volatile("");
        const unsigned base = (unsigned)(qb + 32 * mt + 4 * hi - qs_lane);
        const unsigned lim = (unsigned)max(g.nq - qs_lane, 0);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (base + (unsigned)(8 * (r >> 2) + (r & 3)) >= lim) sc[r] = -INFINITY;
      }
      bf16x8 pb[2], db[2], dl[kSplit ? 2 : 1];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        f32x8 tp, tds;
#pragma unroll
        for (int rg2 = 0; rg2 < 2; ++rg2) {
          const int rg = 2 * s2 + rg2;
          const int qr0 = 32 * mt + 8 * rg + 4 * hi;
          const f32x4 l4 = *(const f32x4*)&sL[qr0];
          const f32x4 d4 = *(const f32x4*)&sD[qr0];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * rg + e;
            const float pr = fast_exp2(__builtin_fmaf(sc[r], c2, -l4[e]));
            tp[4 * rg2 + e] = pr;
            tds[4 * rg2 + e] = pr * (dp[r] - d4[e]);
          }
        }
        pb[s2] = to_bf16x8(tp);
        db[s2] = to_bf16x8(tds);
        if constexpr (kSplit) dl[s2] = lo_half(tds, db[s2]);
      }
      __builtin_amdgcn_sched_barrier(0);
      if (mt == 0) load_s(1);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dvacc[dt] = mfma32(ot[s2][dt], pb[s2], dvacc[dt]);
          dkacc[dt] = mfma32(qt[s2][dt], db[s2], dkacc[dt]);
          if constexpr (kSplit) dkacc[dt] = mfma32(qt[s2][dt], dl[s2], dkacc[dt]);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int s_qt = 0;  // query tile of the next step (the head only matters to the copies)
  auto step = [&](const bf16_t* sQ, const bf16_t* sdO, const float* sL, const float* sD) {
    const int qb = q_begin + s_qt * kBwdBlockQT;
    if (++s_qt == nqt) s_qt = 0;
    if (!wave_active || qb + kBwdBlockQT <= w_qs_min) return;
    compute((qb < w_qs_max) || (qb + kBwdBlockQT > g.nq), qb, sQ, sdO, sL, sD);
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
  // The copies past the last tile (and with n_iter == 0 all loads) are still
  // in flight: none may land in LDS after the workgroup ends.
  wait_vmem();

  if (!wave_active) return;
  const int kpos = ka + l32;
  if (kpos >= g.n) return;
  bf16_t* krow = a.dk + (int64_t)(g.start + kpos) * a.dk_st + (int64_t)hk * a.dk_sh;
  bf16_t* vrow = a.dv + (int64_t)(g.start + kpos) * a.dv_st + (int64_t)hk * a.dv_sh;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 tv;
#pragma unroll
      for (int e = 0; e < 4; ++e) tv[e] = dvacc[dt][4 * rg + e];
      *(bf16x4*)&vrow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tv, bf16x4);
    }
  grad_out<DT>(dkacc, a.scale, a.rope, g.start + kpos, hi,
               [&](int dt, int rg, bf16x4 v) { *(bf16x4*)&krow[32 * dt + 8 * rg + 4 * hi] = v; });
}


// The split body in a function of its own, which the kernel calls when the split
// is on: the plain body, inlined in the kernel, keeps the registers and code of a
// kernel of its own.  It reads its arguments from the kernel's argument segment
// `seg`.
template <int D>
__device__ __attribute__((noinline)) void dkdv_split_body(uint64_t seg) {
  dkdv_body<D, true>(segment_args<BwdArgs>(uniform_segment(seg)));
}
// One launch for every split mode: the decision (the forward's recorded one, or
// the K scan's) picks the body.  The waves per SIMD are pinned as the least and
// the most, so that the called body is scheduled for that occupancy too.
template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(DkCfg<D>::kWaves * 64, DkCfg<D>::kWaves * 64),
                          amdgpu_waves_per_eu(DkCfg<D>::kWavesPerSimd, DkCfg<D>::kWavesPerSimd))) void dkdv_kernel(
    const BwdArgs a) {
  if (split_on(a, threadIdx.x & 63))
    dkdv_split_body<D>(kernel_segment());
  else
    dkdv_body<D, false>(a);
}
template __global__ void dkdv_kernel<64>(const BwdArgs);

template <int D>
hipError_t launch(BwdArgs a, int numseqs, int max_seqlen_all, hipStream_t stream) {
  constexpr int kDkKeys = DkCfg<D>::kKeys, kDkWaves = DkCfg<D>::kWaves;
  static_assert(kDkKeys == kPlanTile, "work-list tiles are the dK / dV key tiles");
  if (numseqs <= 0 || a.cap_k == 0) return hipSuccess;
  // workgroup r * Hkv + h: list entry r, kv head h
  const dim3 grid((unsigned)a.cap_k * (unsigned)a.Hkv);
  hipLaunchKernelGGL(dkdv_kernel<D>, grid, dim3(kDkWaves * 64), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_dkdv_bf16(const BwdArgs& a, int head_dim, int numseqs, int max_seqlen_all,
                                hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch<64>(a, numseqs, max_seqlen_all, stream);
    default: return hipErrorInvalidValue;  // head_dim 128: launch_bwd_dkdv_pair_bf16
  }
}

}  // namespace mimir
