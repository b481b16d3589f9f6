// bf16 prefix-LM attention backward, dK / dV kernel, for gfx950 (MI355X).
// Owner = (kv head, key tile); see prefixlm_bwd_bf16.hip for the split.
#include "prefixlm_bwd_bf16.h"

namespace mimir {
namespace {

// ---------------------------------------------------------------------------
// dK / dV.  Each wave owns kDkSub x 32 keys whose K and V fragments stay in
// registers as B operands; lanes own key columns, so P and dS feed the B operand
// of dV^T += dO^T P and dK^T += Q^T dS directly, and the transposed dO^T / Q^T
// fragments come from the row-major LDS tiles via ds_read_b64_tr_b16.  Every Q /
// dO operand read from LDS (plain or transposed) feeds kSub MFMAs, one per
// 32-key subtile of the wave.
// The query range starts at qstart(first key) = (key < p ? 0 : key).
// Grid: x = sequence * Hkv + kv head, y = key tile (prefix keys, the heaviest, first).
//
// Configuration per head_dim: one 32-key subtile per wave and four waves per
// workgroup measured fastest for both 64 and 128 (two subtiles per wave halve
// the LDS traffic per MFMA but exceed the register file at 128 and spill).
// At 128 the K / V fragments and dK / dV accumulators need one wave per SIMD.
// ---------------------------------------------------------------------------
template <int D>
struct DkCfg {
  static constexpr int kSub = 1;                      // 32-key subtiles per wave
  static constexpr int kWaves = 4;                    // waves per workgroup
  static constexpr int kKeys = 32 * kSub * kWaves;    // keys per workgroup
  static constexpr int kWavesPerSimd = D <= 64 ? 2 : 1;
};

template <int D>
__global__ __launch_bounds__(DkCfg<D>::kWaves * 64, DkCfg<D>::kWavesPerSimd) void dkdv_kernel(const BwdArgs a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  constexpr int NS = DkCfg<D>::kSub;
  constexpr int kDkWaves = DkCfg<D>::kWaves;
  constexpr int kDkKeys = DkCfg<D>::kKeys;
  using L = TileLayout<D>;
  static_assert(kBwdBlockQT == 64, "one TileLayout tile per Q / dO block");
  __shared__ __attribute__((aligned(16))) bf16_t sQ0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sO0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sQ1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sO1[L::kElems];
  __shared__ __attribute__((aligned(16))) float sL0[kBwdBlockQT];
  __shared__ __attribute__((aligned(16))) float sD0[kBwdBlockQT];
  __shared__ __attribute__((aligned(16))) float sL1[kBwdBlockQT];
  __shared__ __attribute__((aligned(16))) float sD1[kBwdBlockQT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  if ((int)blockIdx.x >= a.grid_x) return;
  const int hk = blockIdx.x % a.Hkv;
  const int s = blockIdx.x / a.Hkv;
  const int ktile = blockIdx.y;
  const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int kb0 = ktile * kDkKeys;
  if (kb0 >= g.n) return;

  const int ka = kb0 + wave * 32 * NS;       // this wave's first key
  const bool wave_active = ka < g.n;
  int qs_lane[NS];                           // first query attending this lane's key of subtile j
#pragma unroll
  for (int j = 0; j < NS; ++j) qs_lane[j] = qstart_of(g.p, ka + 32 * j + l32);
  const int w_qs_min = qstart_of(g.p, ka);
  const int w_qs_max = qstart_of(g.p, ka + 32 * NS - 1);
  const int q_begin = qstart_of(g.p, kb0);
  const int nqt = g.nq > q_begin ? (g.nq - q_begin + kBwdBlockQT - 1) / kBwdBlockQT : 0;
  const int n_iter = nqt * a.group;  // (q head, query tile) pairs

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(
      a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh, rows_bytes(g.n, a.k_st, D));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(
      a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh, rows_bytes(g.n, a.v_st, D));

  // Iteration it covers q head hk * G + it / nqt and query tile it % nqt.
  const TileLoader<D, kDkWaves> ldq(a.q_st, wave, lane), ldo(a.do_st, wave, lane);
  auto issue = [&](int it, bf16_t* tq, bf16_t* to, float* tl, float* td) {
    const int hh = it / nqt;
    const int qb = q_begin + (it - hh * nqt) * kBwdBlockQT;
    const int h = hk * a.group + hh;
    ldq.issue(a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, qb, g.nq, tq);
    ldo.issue(a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh, qb, g.nq, to);
    if (wave == 0) {
      const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.lse2 + (int64_t)h * a.T + g.start, (uint32_t)g.nq * 4u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (__attribute__((address_space(3))) void*)tl, 4,
                                               (uint32_t)(qb + lane) * 4u, 0, 0, 0);
    } else {
      const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.delta + (int64_t)h * a.T + g.start, (uint32_t)g.nq * 4u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (__attribute__((address_space(3))) void*)td, 4,
                                               (uint32_t)(qb + lane) * 4u, 0, 0, 0);
    }
  };
  if (n_iter > 0) issue(0, sQ0, sO0, sL0, sD0);

  bf16x8 kf[NS][KS], vf[NS][KS];
#pragma unroll
  for (int j = 0; j < NS; ++j)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int64_t key = ka + 32 * j + l32;
      kf[j][ks] = __builtin_bit_cast(bf16x8, buf_load16(rk, (uint32_t)((key * a.k_st + 16 * ks + 8 * hi) * 2)));
      vf[j][ks] = __builtin_bit_cast(bf16x8, buf_load16(rv, (uint32_t)((key * a.v_st + 16 * ks + 8 * hi) * 2)));
    }

  f32x16 dkacc[NS][DT], dvacc[NS][DT];
#pragma unroll
  for (int j = 0; j < NS; ++j)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      dkacc[j][dt] = f32x16{};
      dvacc[j][dt] = f32x16{};
    }
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  // One (q head, 64-query tile) step.  Masked tiles (queries before some key's
  // qstart, or past the sequence end) overwrite the disallowed scores with -inf
  // in one guarded pass right after the S MFMAs; the softmax and the dV / dK
  // MFMAs that follow are one straight-line block for both kinds of tile.
  auto compute = [&](bool masked, int qb, const bf16_t* sQ, const bf16_t* sdO, const float* sL,
                     const float* sD) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {  // 32-query halves of the tile
      f32x16 sc[NS], dp[NS];
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        sc[j] = f32x16{};
        dp[j] = f32x16{};
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int o = tl.op_base + mt * 32 * L::kRowElems + ks * 16;
        const bf16x8 qa8 = *(const bf16x8*)&sQ[o];
        const bf16x8 da8 = *(const bf16x8*)&sdO[o];
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          sc[j] = mfma32(qa8, kf[j][ks], sc[j]);
          dp[j] = mfma32(da8, vf[j][ks], dp[j]);
        }
      }
      // rows of sc / dp: query 32*mt + 8*(r/4) + 4*hi + r%4 ; column: the lane's key.
      if (masked) {
        // allowed iff qs_lane <= q < nq, i.e. (unsigned)(q - qs_lane) < (unsigned)(nq - qs_lane).
        // The empty volatile asm keeps this block a real branch: if-converted, its
        // 48 VALU operations would run on every unmasked tile as well.
        __asm__ volatile("");
#pragma unroll
        for (int j = 0; j < NS; ++j) {
          const unsigned base = (unsigned)(qb + 32 * mt + 4 * hi - qs_lane[j]);
          const unsigned lim = (unsigned)(g.nq - qs_lane[j]);
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (base + (unsigned)(8 * (r >> 2) + (r & 3)) >= lim) sc[j][r] = -INFINITY;
        }
      }
      // Each 16-query half (s2) is converted to bf16 right before its MFMAs so
      // that its fp32 scores die early.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        bf16x8 pb[NS], db[NS];
#pragma unroll
        for (int j = 0; j < NS; ++j) {
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
              const float pr = fast_exp2(__builtin_fmaf(sc[j][r], c2, -l4[e]));
              tp[4 * rg2 + e] = pr;
              tds[4 * rg2 + e] = pr * (dp[j][r] - d4[e]);
            }
          }
          pb[j] = to_bf16x8(tp);
          db[j] = to_bf16x8(tds);
        }
        const int kk = 2 * mt + s2;  // 16-query step inside the 64-row tile
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int o = tl.tr_base + kk * 16 * L::kRowElems + dt * 32;
          const bf16x8 ot = cat8(lds_read_tr16(&sdO[o]), lds_read_tr16(&sdO[o + L::kTrSecond]));
          const bf16x8 qt = cat8(lds_read_tr16(&sQ[o]), lds_read_tr16(&sQ[o + L::kTrSecond]));
#pragma unroll
          for (int j = 0; j < NS; ++j) {
            dvacc[j][dt] = mfma32(ot, pb[j], dvacc[j][dt]);
            dkacc[j][dt] = mfma32(qt, db[j], dkacc[j][dt]);
          }
        }
      }
    }
  };
  auto step = [&](int it, const bf16_t* sQ, const bf16_t* sdO, const float* sL, const float* sD) {
    const int hh = it / nqt;
    const int qb = q_begin + (it - hh * nqt) * kBwdBlockQT;
    if (!wave_active || qb + kBwdBlockQT <= w_qs_min) return;
    compute((qb < w_qs_max) || (qb + kBwdBlockQT > g.nq), qb, sQ, sdO, sL, sD);
  };

  for (int it = 0; it < n_iter; it += 2) {
    wait_vmem();
    __syncthreads();
    if (it + 1 < n_iter) issue(it + 1, sQ1, sO1, sL1, sD1);
    step(it, sQ0, sO0, sL0, sD0);
    if (it + 1 >= n_iter) break;
    wait_vmem();
    __syncthreads();
    if (it + 2 < n_iter) issue(it + 2, sQ0, sO0, sL0, sD0);
    step(it + 1, sQ1, sO1, sL1, sD1);
  }

  if (!wave_active) return;
#pragma unroll
  for (int j = 0; j < NS; ++j) {
    const int kpos = ka + 32 * j + l32;
    if (kpos >= g.n) continue;
    bf16_t* krow = a.dk + (int64_t)(g.start + kpos) * a.dk_st + (int64_t)hk * a.dk_sh;
    bf16_t* vrow = a.dv + (int64_t)(g.start + kpos) * a.dv_st + (int64_t)hk * a.dv_sh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 tk, tv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          tk[e] = dkacc[j][dt][4 * rg + e] * a.scale;
          tv[e] = dvacc[j][dt][4 * rg + e];
        }
        *(bf16x4*)&krow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tk, bf16x4);
        *(bf16x4*)&vrow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tv, bf16x4);
      }
  }
}


template <int D>
hipError_t launch(BwdArgs a, int numseqs, int max_seqlen_all, hipStream_t stream) {
  constexpr int kDkKeys = DkCfg<D>::kKeys, kDkWaves = DkCfg<D>::kWaves;
  a.num_tiles = (max_seqlen_all + kDkKeys - 1) / kDkKeys;
  if (numseqs <= 0 || a.num_tiles == 0) return hipSuccess;
  a.grid_x = a.Hkv * numseqs;
  hipLaunchKernelGGL(dkdv_kernel<D>, dim3(xcd_spread_width(a.grid_x), a.num_tiles), dim3(kDkWaves * 64), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_bwd_dkdv_bf16(const BwdArgs& a, int head_dim, int numseqs, int max_seqlen_all,
                                hipStream_t stream) {
  switch (head_dim) {
    case 64: return launch<64>(a, numseqs, max_seqlen_all, stream);
    case 128: return launch<128>(a, numseqs, max_seqlen_all, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace mimir
