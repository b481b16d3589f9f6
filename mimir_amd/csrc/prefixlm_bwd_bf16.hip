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
// Math: dV = P^T dO, dP = dO V^T, delta = rowsum(dO * O), dS = P (dP - delta) * scale,
// dQ = dS K, dK = dS^T Q  (flash_attention_prefixlm_mps.py:1601-1675), with the GQA
// head map of flash_attention_prefixlm_dense.py:10-16 (q head h -> kv head h / G).
#include "prefixlm_common.h"

namespace {
using namespace mimir;

constexpr int kThreads = 256;
constexpr int kBlockQ = 128;  // dq: query rows per workgroup (32 per wave)
constexpr int kBlockK = 64;   // dq: keys per LDS tile
constexpr int kBlockKV = 128; // dkdv: keys per workgroup (32 per wave)
constexpr int kBlockQT = 64;  // dkdv: query rows per LDS tile

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
  int group;
  int total_seqlen;
  int is_causal;
  int num_q_tiles;   // dq grid
  int num_kv_tiles;  // dkdv grid
  float scale;
  float scale_log2;
};

__device__ __forceinline__ uint32_t rows_bytes(int rows, int64_t stride, int d) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * stride + d) * 2) : 0u;
}

// ---------------------------------------------------------------------------
// delta = rowsum(O * dO), one (token, head) row per D/8 lanes.
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void delta_kernel(const BwdArgs a) {
  constexpr int LPR = D / 8;  // lanes per row
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int row = gid / LPR;  // row = t * Hq + h
  const int c = gid % LPR;
  const bool valid = row < a.T * a.Hq;
  const int t = valid ? row / a.Hq : 0;
  const int h = valid ? row % a.Hq : 0;
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
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads, 1) void dq_kernel(const BwdArgs a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  constexpr int CPR = D / 8;
  constexpr int LOADS = kBlockK * CPR / kThreads;
  __shared__ __attribute__((aligned(16))) bf16_t sK[kBlockK * D];
  __shared__ __attribute__((aligned(16))) bf16_t sV[kBlockK * D];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int h = blockIdx.x;
  const int qtile = a.num_q_tiles - 1 - (int)blockIdx.y;
  const int s = blockIdx.z;
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
  const int tj = lane & 15, tg = lane >> 4, t_hi = tg >> 1, t_dh = tg & 1;

  for (int kt = 0; kt < nkt; ++kt) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int idx = tid + i * kThreads;
      const int row = idx / CPR, c = idx % CPR;
      const int key = kt * kBlockK + row;
      *(i32x4*)&sK[swz<D>(row, c * 8)] = buf_load16(rk, (uint32_t)(((int64_t)key * a.k_st + c * 8) * 2));
      *(i32x4*)&sV[swz<D>(row, c * 8)] = buf_load16(rv, (uint32_t)(((int64_t)key * a.v_st + c * 8) * 2));
    }
    __syncthreads();
    const int kb = kt * kBlockK;
    if (!wave_active || kb >= w_kend_max) continue;

    f32x16 st[2], dpt[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = f32x16{};
      dpt[mt] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kf = *(const bf16x8*)&sK[swz<D>(32 * mt + l32, 16 * ks + 8 * hi)];
        const bf16x8 vf = *(const bf16x8*)&sV[swz<D>(32 * mt + l32, 16 * ks + 8 * hi)];
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
      const int col = 32 * dt + 16 * t_dh + 4 * (tj & 3);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int krow = 16 * kk + 4 * t_hi + (tj >> 2);
        const bf16x4 k0 = lds_read_tr16(&sK[swz<D>(krow, col)]);
        const bf16x4 k1 = lds_read_tr16(&sK[swz<D>(krow + 8, col)]);
        dqacc[dt] = mfma32(cat8(k0, k1), sf[kk], dqacc[dt]);
      }
    }
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
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kThreads, 1) void dkdv_kernel(const BwdArgs a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  constexpr int CPR = D / 8;
  constexpr int LOADS = kBlockQT * CPR / kThreads;
  __shared__ __attribute__((aligned(16))) bf16_t sQ[kBlockQT * D];
  __shared__ __attribute__((aligned(16))) bf16_t sdO[kBlockQT * D];
  __shared__ __attribute__((aligned(16))) float sL[kBlockQT];
  __shared__ __attribute__((aligned(16))) float sD[kBlockQT];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hi = lane >> 5;
  const int hk = blockIdx.x;
  const int ktile = blockIdx.y;
  const int s = blockIdx.z;
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

  const __amdgpu_buffer_rsrc_t rk = make_rsrc(
      a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh, rows_bytes(g.n, a.k_st, D));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(
      a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh, rows_bytes(g.n, a.v_st, D));
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
  const int tj = lane & 15, tg = lane >> 4, t_hi = tg >> 1, t_dh = tg & 1;

  for (int hh = 0; hh < a.group; ++hh) {
    const int h = hk * a.group + hh;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(
        a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, rows_bytes(g.nq, a.q_st, D));
    const __amdgpu_buffer_rsrc_t rdo = make_rsrc(
        a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh, rows_bytes(g.nq, a.do_st, D));
    const float* lse_h = a.lse + (int64_t)h * a.lse_sh + g.start;
    const float* dl_h = a.delta + (int64_t)h * a.T + g.start;

    for (int qt = 0; qt < nqt; ++qt) {
      const int qb = q_begin + qt * kBlockQT;
      __syncthreads();
#pragma unroll
      for (int i = 0; i < LOADS; ++i) {
        const int idx = tid + i * kThreads;
        const int row = idx / CPR, c = idx % CPR;
        const int qr = qb + row;
        *(i32x4*)&sQ[swz<D>(row, c * 8)] = buf_load16(rq, (uint32_t)(((int64_t)qr * a.q_st + c * 8) * 2));
        *(i32x4*)&sdO[swz<D>(row, c * 8)] = buf_load16(rdo, (uint32_t)(((int64_t)qr * a.do_st + c * 8) * 2));
      }
      if (tid < kBlockQT) {
        const int qr = qb + tid;
        const bool ok = qr < g.nq;
        sL[tid] = ok ? lse_h[qr] * kLog2e : 0.f;
        sD[tid] = ok ? dl_h[qr] : 0.f;
      }
      __syncthreads();
      if (!wave_active || qb + kBlockQT <= w_qs_min) continue;
      const bool masked = (qb < w_qs_max) || (qb + kBlockQT > g.nq);

#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        f32x16 sc = f32x16{}, dp = f32x16{};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 qa8 = *(const bf16x8*)&sQ[swz<D>(32 * mt + l32, 16 * ks + 8 * hi)];
          const bf16x8 da8 = *(const bf16x8*)&sdO[swz<D>(32 * mt + l32, 16 * ks + 8 * hi)];
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
            float pr = fast_exp2(__builtin_fmaf(sc[r], c2, -l4[e]));
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
            const int col = 32 * dt + 16 * t_dh + 4 * (tj & 3);
            const int qrow = 16 * kk + 4 * t_hi + (tj >> 2);
            const bf16x4 o0 = lds_read_tr16(&sdO[swz<D>(qrow, col)]);
            const bf16x4 o1 = lds_read_tr16(&sdO[swz<D>(qrow + 8, col)]);
            dvacc[dt] = mfma32(cat8(o0, o1), pb, dvacc[dt]);
            const bf16x4 q0 = lds_read_tr16(&sQ[swz<D>(qrow, col)]);
            const bf16x4 q1 = lds_read_tr16(&sQ[swz<D>(qrow + 8, col)]);
            dkacc[dt] = mfma32(cat8(q0, q1), db, dkacc[dt]);
          }
        }
      }
    }
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
      hipLaunchKernelGGL(dkdv_kernel<D>, dim3(p.num_kv_heads, a.num_kv_tiles, p.numseqs), dim3(kThreads), 0,
                         stream, a);
    if (stages & MIMIR_BWD_STAGE_DQ)
      hipLaunchKernelGGL(dq_kernel<D>, dim3(p.num_q_heads, a.num_q_tiles, p.numseqs), dim3(kThreads), 0,
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
