// bf16 prefix-LM attention backward for gfx950 (MI355X): an atomic-free split
// into three kernels, the same ownership split as the reference's Metal
// backward (flash_attention_prefixlm_mps.py:867-898 delta, 967-1039 dQ per query
// row, 1245-1322 dK/dV per key row), re-tiled for bf16 MFMA.
//
//   delta:  delta[h, t] = sum_d O[t, h, d] * dO[t, h, d]                 (fp32)
//   dq:     owner = (query head, 128 query rows).  Per 64-key tile:
//             S^T = K Q^T, dP^T = V dO^T, P^T = exp(scale*S^T - lse),
//             dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.
//   dkdv:   owner = (kv head, 128 keys).  Per q-head of the GQA group and per
//           64-query tile:  S = Q K^T, dP = dO V^T, P, dS as above,
//             dV^T += dO^T P,  dK^T += Q^T dS.
//           The GQA reduction over the q-heads of one kv head happens in
//           registers, so no kernel needs atomics and results are deterministic.
//
// Both tile loops stream their operand tiles with direct buffer-to-LDS loads
// into two LDS stages (one barrier per tile).  Grids are ordered so that the
// heaviest tiles of every sequence are dispatched first.
//
// Math: dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta) * scale,
// dQ = dS K, dK = dS^T Q  (flash_attention_prefixlm_mps.py:1601-1675), with the GQA
// head map of flash_attention_prefixlm_dense.py:10-16 (q head h -> kv head h / G).
#include "prefixlm_common.h"

namespace {
using namespace mimir;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBlockQ = 128;   // dq: query rows per workgroup (32 per wave)
constexpr int kBlockK = 64;    // dq: keys per LDS tile
constexpr int kBlockKV = 128;  // dkdv: keys per workgroup (32 per wave)
constexpr int kBlockQT = 64;   // dkdv: query rows per LDS tile

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
  float* delta;
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
  int num_q_tiles;   // dq grid
  int num_kv_tiles;  // dkdv grid
  float scale;
  float scale_log2;
};

// ---------------------------------------------------------------------------
// delta = rowsum(O * dO), one (token, head) row per D/8 lanes.
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
  if (valid && c == 0) a.delta[(int64_t)h * a.T + t] = acc;
}

// ---------------------------------------------------------------------------
// dQ.  Mirrors the forward's S^T formulation: each lane owns one query column,
// so lse and delta are lane-local and dS^T feeds the B operand of dQ^T += K^T dS^T
// directly; K^T fragments come from the row-major K tile via ds_read_b64_tr_b16.
// Grid: x = sequence * Hq + head, y = query tile (reversed: longest key ranges first).
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads, 2) void dq_kernel(const BwdArgs a) {
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
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int h = blockIdx.x % a.Hq;
  const int s = blockIdx.x / a.Hq;
  const int qtile = a.num_q_tiles - 1 - (int)blockIdx.y;
  const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = qtile * kBlockQ;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;

  const int wg_kend = max(g.p, min(m0 + kBlockQ, g.nq));
  const int nkt = (wg_kend + kBlockK - 1) / kBlockK;
  const int qa = m0 + wave * 32;
  const bool wave_active = qa < g.nq;
  const int w_kend_max = wave_active ? max(g.p, min(qa + 32, g.nq)) : 0;
  const int w_kend_min = max(g.p, qa + 1);
  const int qpos = qa + l32;
  const int kend_lane = kend_of(g.p, qpos);

  const __amdgpu_buffer_rsrc_t rq =
      make_rsrc(a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, rows_bytes(g.nq, a.q_st, D));
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc(
      a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh, rows_bytes(g.nq, a.do_st, D));
  const __amdgpu_buffer_rsrc_t rk =
      make_rsrc(a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh, rows_bytes(g.n, a.k_st, D));
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh, rows_bytes(g.n, a.v_st, D));

  auto issue = [&](int kt, bf16_t* tk, bf16_t* tv) {
    lds_tile_async<D, kWaves>(rk, a.k_st, kt * kBlockK, tk, wave, lane);
    lds_tile_async<D, kWaves>(rv, a.v_st, kt * kBlockK, tv, wave, lane);
  };
  issue(0, sK0, sV0);

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
    const bool masked = kb + kBlockK > w_kend_min;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kpos = kb + 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
        float pr = fast_exp2(__builtin_fmaf(st[mt][r], c2, -lse2));
        if (masked && kpos >= kend_lane) pr = 0.f;
        st[mt][r] = pr * (dpt[mt][r] - dlt);
      }
    bf16x8 sf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int mt = kk >> 1, s8 = (kk & 1) * 8;
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = st[mt][s8 + e];
      sf[kk] = to_bf16x8(t);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16_t* kp = &sK[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
        const bf16x4 k0 = lds_read_tr16(kp);
        const bf16x4 k1 = lds_read_tr16(kp + 8 * L::kRowElems);
        dqacc[dt] = mfma32(cat8(k0, k1), sf[kk], dqacc[dt]);
      }
    }
  };

  for (int kt = 0; kt < nkt; kt += 2) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < nkt) issue(kt + 1, sK1, sV1);
    compute(kt, sK0, sV0);
    if (kt + 1 >= nkt) break;
    wait_vmem();
    __syncthreads();
    if (kt + 2 < nkt) issue(kt + 2, sK0, sV0);
    compute(kt + 1, sK1, sV1);
  }

  if (!wave_active || qpos >= g.nq) return;
  bf16_t* drow = a.dq + (int64_t)(g.start + qpos) * a.dq_st + (int64_t)h * a.dq_sh;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 t;
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = dqacc[dt][4 * rg + e] * a.scale;
      *(bf16x4*)&drow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(t, bf16x4);
    }
}

// ---------------------------------------------------------------------------
// dK / dV.  Each wave owns 32 keys whose K and V fragments stay in registers as
// B operands; lanes own key columns, so P and dS feed the B operand of
// dV^T += dO^T P and dK^T += Q^T dS directly, and the transposed dO^T / Q^T
// fragments come from the row-major LDS tiles via ds_read_b64_tr_b16.
// The query range starts at qstart(first key) = (key < p ? 0 : key).
// Grid: x = sequence * Hkv + kv head, y = key tile (prefix keys, the heaviest, first).
// ---------------------------------------------------------------------------
// Two waves per SIMD fit the register budget at head_dim 64; at 128 the K / V
// fragments plus the dK / dV accumulators need one wave per SIMD.
template <int D>
__global__ __launch_bounds__(kThreads, D <= 64 ? 2 : 1) void dkdv_kernel(const BwdArgs a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  using L = TileLayout<D>;
  static_assert(kBlockQT == 64, "one TileLayout tile per Q / dO block");
  __shared__ __attribute__((aligned(16))) bf16_t sQ0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sO0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sQ1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sO1[L::kElems];
  __shared__ __attribute__((aligned(16))) float sL0[kBlockQT];
  __shared__ __attribute__((aligned(16))) float sD0[kBlockQT];
  __shared__ __attribute__((aligned(16))) float sL1[kBlockQT];
  __shared__ __attribute__((aligned(16))) float sD1[kBlockQT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int hk = blockIdx.x % a.Hkv;
  const int s = blockIdx.x / a.Hkv;
  const int ktile = blockIdx.y;
  const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int kb0 = ktile * kBlockKV;
  if (kb0 >= g.n) return;

  const int ka = kb0 + wave * 32;            // this wave's first key
  const bool wave_active = ka < g.n;
  const int kpos = ka + l32;                 // this lane's key
  const int qs_lane = qstart_of(g.p, kpos);  // first query attending this key
  const int w_qs_min = qstart_of(g.p, ka);
  const int w_qs_max = qstart_of(g.p, ka + 31);
  const int q_begin = qstart_of(g.p, kb0);
  const int nqt = g.nq > q_begin ? (g.nq - q_begin + kBlockQT - 1) / kBlockQT : 0;
  const int n_iter = nqt * a.group;  // (q head, query tile) pairs

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(
      a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh, rows_bytes(g.n, a.k_st, D));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(
      a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh, rows_bytes(g.n, a.v_st, D));

  // Iteration it covers q head hk * G + it / nqt and query tile it % nqt.
  auto issue = [&](int it, bf16_t* tq, bf16_t* to, float* tl, float* td) {
    const int hh = it / nqt;
    const int qb = q_begin + (it - hh * nqt) * kBlockQT;
    const int h = hk * a.group + hh;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, rows_bytes(g.nq, a.q_st, D));
    const __amdgpu_buffer_rsrc_t rdo = make_rsrc(
        a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh, rows_bytes(g.nq, a.do_st, D));
    lds_tile_async<D, kWaves>(rq, a.q_st, qb, tq, wave, lane);
    lds_tile_async<D, kWaves>(rdo, a.do_st, qb, to, wave, lane);
    if (wave == 0) {
      const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.lse + (int64_t)h * a.lse_sh + g.start, (uint32_t)g.nq * 4u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, (__attribute__((address_space(3))) void*)tl, 4,
                                               (uint32_t)(qb + lane) * 4u, 0, 0, 0);
    } else if (wave == 1) {
      const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.delta + (int64_t)h * a.T + g.start, (uint32_t)g.nq * 4u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rd, (__attribute__((address_space(3))) void*)td, 4,
                                               (uint32_t)(qb + lane) * 4u, 0, 0, 0);
    }
  };
  if (n_iter > 0) issue(0, sQ0, sO0, sL0, sD0);

  bf16x8 kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rk, (uint32_t)(((int64_t)kpos * a.k_st + 16 * ks + 8 * hi) * 2)));
    vf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rv, (uint32_t)(((int64_t)kpos * a.v_st + 16 * ks + 8 * hi) * 2)));
  }

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = f32x16{};
    dvacc[dt] = f32x16{};
  }
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  auto compute = [&](int it, const bf16_t* sQ, const bf16_t* sdO, const float* sL, const float* sD) {
    const int hh = it / nqt;
    const int qb = q_begin + (it - hh * nqt) * kBlockQT;
    if (!wave_active || qb + kBlockQT <= w_qs_min) return;
    const bool masked = (qb < w_qs_max) || (qb + kBlockQT > g.nq);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      f32x16 sc = f32x16{}, dp = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int o = tl.op_base + mt * 32 * L::kRowElems + ks * 16;
        const bf16x8 qa8 = *(const bf16x8*)&sQ[o];
        const bf16x8 da8 = *(const bf16x8*)&sdO[o];
        sc = mfma32(qa8, kf[ks], sc);
        dp = mfma32(da8, vf[ks], dp);
      }
      // rows of sc / dp: query 32*mt + 8*(r/4) + 4*hi + r%4 ; column: this lane's key
      f32x16 pm, ds;
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        const int qr0 = 32 * mt + 8 * rg + 4 * hi;
        const f32x4 l4 = *(const f32x4*)&sL[qr0];
        const f32x4 d4 = *(const f32x4*)&sD[qr0];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * rg + e;
          float pr = fast_exp2(__builtin_fmaf(sc[r], c2, -l4[e] * kLog2e));
          if (masked) {
            const int qp = qb + qr0 + e;
            if (qp < qs_lane || qp >= g.nq) pr = 0.f;
          }
          pm[r] = pr;
          ds[r] = pr * (dp[r] - d4[e]);
        }
      }
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        f32x8 tp, tds;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          tp[e] = pm[8 * s2 + e];
          tds[e] = ds[8 * s2 + e];
        }
        const bf16x8 pb = to_bf16x8(tp);
        const bf16x8 db = to_bf16x8(tds);
        const int kk = 2 * mt + s2;  // 16-query step inside the 64-row tile
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int o = tl.tr_base + kk * 16 * L::kRowElems + dt * 32;
          const bf16x4 o0 = lds_read_tr16(&sdO[o]);
          const bf16x4 o1 = lds_read_tr16(&sdO[o + 8 * L::kRowElems]);
          dvacc[dt] = mfma32(cat8(o0, o1), pb, dvacc[dt]);
          const bf16x4 q0 = lds_read_tr16(&sQ[o]);
          const bf16x4 q1 = lds_read_tr16(&sQ[o + 8 * L::kRowElems]);
          dkacc[dt] = mfma32(cat8(q0, q1), db, dkacc[dt]);
        }
      }
    }
  };

  for (int it = 0; it < n_iter; it += 2) {
    wait_vmem();
    __syncthreads();
    if (it + 1 < n_iter) issue(it + 1, sQ1, sO1, sL1, sD1);
    compute(it, sQ0, sO0, sL0, sD0);
    if (it + 1 >= n_iter) break;
    wait_vmem();
    __syncthreads();
    if (it + 2 < n_iter) issue(it + 2, sQ0, sO0, sL0, sD0);
    compute(it + 1, sQ1, sO1, sL1, sD1);
  }

  if (!wave_active || kpos >= g.n) return;
  bf16_t* krow = a.dk + (int64_t)(g.start + kpos) * a.dk_st + (int64_t)hk * a.dk_sh;
  bf16_t* vrow = a.dv + (int64_t)(g.start + kpos) * a.dv_st + (int64_t)hk * a.dv_sh;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 tk, tv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tk[e] = dkacc[dt][4 * rg + e] * a.scale;
        tv[e] = dvacc[dt][4 * rg + e];
      }
      *(bf16x4*)&krow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tk, bf16x4);
      *(bf16x4*)&vrow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(tv, bf16x4);
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
  a.num_q_tiles = (p.max_seqlen_all + kBlockQ - 1) / kBlockQ;
  a.num_kv_tiles = (p.max_seqlen_all + kBlockKV - 1) / kBlockKV;
  a.scale = p.softmax_scale;
  a.scale_log2 = p.softmax_scale * kLog2e;

  const int64_t rows = (int64_t)p.total_tokens * p.num_q_heads;
  if (rows > 0 && (stages & MIMIR_BWD_STAGE_DELTA)) {
    const int64_t threads = rows * (D / 8);
    hipLaunchKernelGGL(delta_kernel<D>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, a);
  }
  if (p.numseqs > 0 && a.num_q_tiles > 0) {
    if (stages & MIMIR_BWD_STAGE_DKDV)
      hipLaunchKernelGGL(dkdv_kernel<D>, dim3(p.num_kv_heads * p.numseqs, a.num_kv_tiles), dim3(kThreads), 0,
                         stream, a);
    if (stages & MIMIR_BWD_STAGE_DQ)
      hipLaunchKernelGGL(dq_kernel<D>, dim3(p.num_q_heads * p.numseqs, a.num_q_tiles), dim3(kThreads), 0,
                         stream, a);
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
