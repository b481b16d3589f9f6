// bf16 prefix-LM attention backward, dQ kernel, for gfx950 (MI355X).
// Owner = (query head, 128 query rows); see prefixlm_bwd_bf16.hip for the split.
#include "prefixlm_bwd_bf16.h"

namespace mimir {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBlockQ = 128;  // query rows per workgroup (32 per wave)
constexpr int kBlockK = 64;   // keys per LDS tile

// ---------------------------------------------------------------------------
// dQ.  Mirrors the forward's S^T formulation: each lane owns one query column,
// so lse and delta are lane-local and dS^T feeds the B operand of dQ^T += K^T dS^T
// directly; K^T fragments come from the row-major K tile via ds_read_b64_tr_b16.
// Workgroup b = r * Hq + h takes head h of entry r of the query-tile work list
// (prefixlm_prologue.hip): longest key ranges first.
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ void dq_tiles(const BwdArgs& a, int b) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  using L = TileLayout<D>;
  static_assert(kBlockK == 64, "one TileLayout tile per K / V block");
  __shared__ __attribute__((aligned(16))) bf16_t sK0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sK1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV1[L::kElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int rank = b / a.Hq;
  const int h = b - rank * a.Hq;
  const int4 item = load_entry(a.plan, rank);
  if (item.x < 0) return;  // list padding
  const int s = item.x;
  const int qtile = item.y;
  const int part = item.z & 0xff, parts = (item.z >> 8) & 0xff, span = item.z >> 16;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = qtile * kBlockQ;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;
  // dS split into bf16 hi + lo for the dQ product (wave-uniform)
  const bool split = split_on(a, lane);

  const int wg_kend = max(g.p, min(m0 + kBlockQ, g.nq));
  const int nkt_all = (wg_kend + kBlockK - 1) / kBlockK;
  // key tiles [kt0, nkt) of this part: the whole range unless the list cut it, then
  // the last parts `span` tiles each and the first the rest
  const int kt0 = part == 0 ? 0 : nkt_all - (parts - part) * span;
  const int nkt = nkt_all - (parts - 1 - part) * span;
  const int qa = m0 + wave * 32;
  const bool wave_active = qa < g.nq;
  const int w_kend_max = wave_active ? max(g.p, min(qa + 32, g.nq)) : 0;
  const int w_kend_min = max(g.p, qa + 1);
  const int qpos = qa + l32;

  const __amdgpu_buffer_rsrc_t rq =
      make_rsrc(a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, rows_bytes(g.nq, a.q_st, D));
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc(
      a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh, rows_bytes(g.nq, a.do_st, D));
  const bf16_t* kseq = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const bf16_t* vseq = a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh;
  const TileLoader<D, kWaves> ldk(a.k_st, wave, lane), ldv(a.v_st, wave, lane);

  // Tile copies walk the key tiles in order with running addresses (adds only).
  const bf16_t* i_k = kseq + (int64_t)kt0 * kBlockK * a.k_st;
  const bf16_t* i_v = vseq + (int64_t)kt0 * kBlockK * a.v_st;
  int i_rows = g.n - kt0 * kBlockK;
  auto issue_next = [&](bf16_t* tk, bf16_t* tv) {
    ldk.issue_at(i_k, rows_bytes32(i_rows, (uint32_t)a.k_st, D), tk);
    ldv.issue_at(i_v, rows_bytes32(i_rows, (uint32_t)a.v_st, D), tv);
    i_k += kBlockK * a.k_st;
    i_v += kBlockK * a.v_st;
    i_rows -= kBlockK;
  };
  if (kt0 < nkt) issue_next(sK0, sV0);

  bf16x8 qf[KS], dof[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, (uint32_t)(((int64_t)qpos * a.q_st + 16 * ks + 8 * hi) * 2)));
    dof[ks] = __builtin_bit_cast(bf16x8, buf_load16(rdo, (uint32_t)(((int64_t)qpos * a.do_st + 16 * ks + 8 * hi) * 2)));
  }
  float lse2 = 0.f, dlt = 0.f;
  if (qpos < g.nq) {
    lse2 = a.lse[(int64_t)h * a.lse_sh + g.start + qpos] * kLog2e;
    dlt = a.delta[(int64_t)h * a.T + g.start + qpos];
  }

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = f32x16{};
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  auto compute = [&](int kt, const bf16_t* sK, const bf16_t* sV) {
    const int kb = kt * kBlockK;
    if (!wave_active || kb >= w_kend_max) return;
    f32x16 st[2], dpt[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = f32x16{};
      dpt[mt] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int o = tl.op_base + mt * 32 * L::kRowElems + ks * 16;
        const bf16x8 kf = *(const bf16x8*)&sK[o];
        const bf16x8 vf = *(const bf16x8*)&sV[o];
        st[mt] = mfma32(kf, qf[ks], st[mt]);
        dpt[mt] = mfma32(vf, dof[ks], dpt[mt]);
      }
    }
    if (kb + kBlockK > w_kend_min) {
      // Tile reaches past some row's kend: disallowed scores become -inf (P = 0).
      // The empty volatile asm keeps this a real branch, so unmasked tiles do not
      // pay for the compares.
      __asm__ volatile("");
      // kpos >= kend(qpos) with kpos = kb + 32 mt + 8 (r / 4) + 4 hi + r % 4; the
      // lane terms are rebuilt here rather than kept in a register across the loop
      const int ln = opaque_lane_id();
      const int base = kb + 4 * (ln >> 5) - kend_of(g.p, qa + (ln & 31));
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (base + 32 * mt + 8 * (r >> 2) + (r & 3) >= 0) st[mt][r] = -INFINITY;
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(__builtin_fmaf(st[mt][r], c2, -lse2));
        st[mt][r] = pr * (dpt[mt][r] - dlt);
      }
    // dQ^T += K^T dS^T; split: dS = hi + lo with lo = round(dS - hi), one more
    // MFMA per K^T fragment (the rounding of dS then no longer reaches dQ).
    bf16x8 sf[4], sl[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int mt = kk >> 1, s8 = (kk & 1) * 8;
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = st[mt][s8 + e];
      sf[kk] = to_bf16x8(t);
      if (split) {
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] -= (float)sf[kk][e];
        sl[kk] = to_bf16x8(t);
      }
    }
    auto dq_mfmas = [&](auto split_tag) {
      constexpr bool kSplit = decltype(split_tag)::value;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16_t* kp = &sK[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
          const bf16x4 k0 = lds_read_tr16(kp);
          const bf16x4 k1 = lds_read_tr16(kp + L::kTrSecond);
          const bf16x8 kt = cat8(k0, k1);
          dqacc[dt] = mfma32(kt, sf[kk], dqacc[dt]);
          if constexpr (kSplit) dqacc[dt] = mfma32(kt, sl[kk], dqacc[dt]);
        }
      }
    };
    if (split)
      dq_mfmas(BoolTag<true>{});
    else
      dq_mfmas(BoolTag<false>{});
  };

  for (int kt = kt0; kt < nkt; kt += 2) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < nkt) issue_next(sK1, sV1);
    compute(kt, sK0, sV0);
    if (kt + 1 >= nkt) break;
    wait_vmem();
    __syncthreads();
    if (kt + 2 < nkt) issue_next(sK0, sV0);
    compute(kt + 1, sK1, sV1);
  }

  // A part of a cut key range: the last part of the tile to arrive sums them.
  if (__builtin_expect(parts > 1, 0) && !dq_merge_parts<DT>(a, kernel_segment(), item, h, wave, lane, dqacc)) return;

  // Epilogue: each wave stages its 32 dQ rows in LDS (one K / V stage object
  // per wave, free once every wave is past the tile loop) and stores whole
  // rows: kRowsPerInst rows of D * 2 contiguous bytes per instruction.
  __syncthreads();
  if (!wave_active) return;
  constexpr int kPitch = D + 8;  // elements; rows stay 16-byte aligned
  constexpr int kUnits = D / 8;  // 16-byte units per row
  constexpr int kRowsPerInst = 64 / kUnits;
  static_assert(32 * kPitch <= L::kElems, "a wave's rows fit its stage object");
  bf16_t* const stage = wave == 0 ? sK0 : wave == 1 ? sV0 : wave == 2 ? sK1 : sV1;
  grad_out<DT>(dqacc, a.scale, a.rope, min(g.start + qa + l32, a.T - 1), hi, [&](int dt, int rg, bf16x4 v) {
    *(bf16x4*)&stage[l32 * kPitch + 32 * dt + 8 * rg + 4 * hi] = v;
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

template <int D>
__global__ __launch_bounds__(kThreads, 2) void dq_kernel(const BwdArgs a) {
  dq_tiles<D>(a, blockIdx.x);
}

// The launch beside the score-gradient hand-off's dQ (head_dim 128), which works
// only when the hand-off cannot (dS split, or a tile that did not fit the
// region).  It checks that first, so that when it has nothing to do its
// workgroups exit after one round of loads instead of three dependent ones (list
// entry, sequence, flags).  (A grid of one resident round looping over the
// entries would exit sooner still, but the loop spills ~50 registers in the
// work it does when the hand-off is ruled out.)
__global__ __launch_bounds__(kThreads, 2) void dq_companion_kernel(const BwdArgs a) {
  // The flags are read with atomic loads, which are not merged with the body's
  // reads of them: a decision kept live across the body cost it a register spill.
  auto flag = [](const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
  bool work = a.split_mode == MIMIR_SPLIT_ALWAYS || flag(&a.queue[kDsIncomplete]) != 0;
  if (!work && a.split_mode == MIMIR_SPLIT_AUTO) {
    if (a.split_flag != nullptr) {
      work = flag(a.split_flag) != 0;
    } else {
      const int lane = threadIdx.x & 63;
      int any = 0;
#pragma unroll
      for (int i = 0; i < kKScanSlots / 64; ++i) any |= flag(&a.kscan[i * 64 + lane]);
      work = __builtin_amdgcn_ballot_w64(any != 0) != 0;
    }
  }
  if (!work) return;
  dq_tiles<128>(a, blockIdx.x);
}

template <int D, bool kCompanion = false>
hipError_t launch(BwdArgs a, int numseqs, int max_seqlen_all, hipStream_t stream) {
  static_assert(kBlockQ == kPlanTile, "work-list tiles are the dQ query tiles");
  if (numseqs <= 0 || a.cap_q == 0) return hipSuccess;
  // workgroup r * Hq + h: list entry r, head h
  static_assert(!kCompanion || D == 128, "the companion serves the head_dim 128 hand-off");
  hipLaunchKernelGGL(kCompanion ? dq_companion_kernel : dq_kernel<D>, dim3((unsigned)a.cap_q * (unsigned)a.Hq),
                     dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}


}  // namespace

hipError_t launch_bwd_dq_bf16(const BwdArgs& a, int head_dim, int numseqs, int max_seqlen_all, hipStream_t stream) {
  if (head_dim == 128 && a.dscore != nullptr) {
    // dQ from the stored tiles, and beside it the recomputing kernel, which
    // works only when the device-side checks rule the stored tiles out (dS split,
    // or a tile that did not fit the region); otherwise its workgroups exit at once.
    hipError_t e = launch_bwd_dq_ds_bf16(a, numseqs, stream);
    if (e != hipSuccess) return e;
    return launch<128, true>(a, numseqs, max_seqlen_all, stream);
  }
  switch (head_dim) {
    case 64: return launch<64>(a, numseqs, max_seqlen_all, stream);
    case 128: return launch<128>(a, numseqs, max_seqlen_all, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mimir
