// float32 prefix-LM attention (forward + backward) for gfx950.
//
// The fp32 path serves the reference's CPU training precision
// (flash_attention_prefixlm_dense.py runs in fp32) and is held to the fp32
// oracle at 1e-5, so it keeps every product and sum in fp32 on the vector ALUs:
// four lanes share one row (D/4 contiguous values each; eight in the forward) and
// combine dot products with cross-lane adds.  K/V (forward, dQ) or Q/dO (dK/dV) tiles are staged in
// LDS and read as broadcasts.  Structure and ownership follow the Metal kernels
// of flash_attention_prefixlm_mps.py (forward 391-476, dQ 967-1039, dK/dV
// 1245-1322), extended to GQA.
#include "prefixlm_common.h"

namespace {
using namespace mimir;

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 4;  // 64 rows, 4 lanes per row
constexpr int kTile = 32;                    // keys (or queries) per LDS tile

struct F32Args {
  const float* q;
  const float* k;
  const float* v;
  float* o;
  float* lse;
  const float* olse;  // bwd: forward lse
  const float* out;   // bwd: forward output
  const float* dout;
  float* dq;
  float* dk;
  float* dv;
  float* delta;
  const int32_t* prefix_lens;
  const int32_t* cu_seqlens;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, do_st, do_sh;
  int64_t dq_st, dq_sh, dk_st, dk_sh, dv_st, dv_sh, lse_sh;
  int T, Hq, Hkv, group, total_seqlen, is_causal, num_tiles;
  float scale, scale_log2;
};

__device__ __forceinline__ float sum4(float x) {
  x += __shfl_xor(x, 1, 64);
  x += __shfl_xor(x, 2, 64);
  return x;
}

template <int D>
__device__ __forceinline__ void load_row(float (&dst)[D / 4], const float* row, int sub, bool valid) {
#pragma unroll
  for (int e = 0; e < D / 4; e += 4) {
    f32x4 t = valid ? *(const f32x4*)&row[sub * (D / 4) + e] : f32x4{0.f, 0.f, 0.f, 0.f};
    dst[e] = t[0]; dst[e + 1] = t[1]; dst[e + 2] = t[2]; dst[e + 3] = t[3];
  }
}

// Cooperative load of `kTile` rows [r0, r0 + kTile) of a [rows][stride] fp32
// matrix into an LDS tile [kTile][D]; rows >= nrows are zero-filled.
template <int D>
__device__ __forceinline__ void stage(float* tile, const float* base, int64_t stride, int r0, int nrows) {
  constexpr int V4 = D / 4;
  for (int i = threadIdx.x; i < kTile * V4; i += kThreads) {
    const int row = i / V4, c = i % V4;
    const int r = r0 + row;
    f32x4 t = r < nrows ? *(const f32x4*)&base[(int64_t)r * stride + 4 * c] : f32x4{0.f, 0.f, 0.f, 0.f};
    *(f32x4*)&tile[row * D + 4 * c] = t;
  }
}

template <int D>
__device__ __forceinline__ float dot_tile(const float (&x)[D / 4], const float* tile_row, int sub) {
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < D / 4; e += 4) {
    const f32x4 t = *(const f32x4*)&tile_row[sub * (D / 4) + e];
    acc = __builtin_fmaf(x[e], t[0], acc);
    acc = __builtin_fmaf(x[e + 1], t[1], acc);
    acc = __builtin_fmaf(x[e + 2], t[2], acc);
    acc = __builtin_fmaf(x[e + 3], t[3], acc);
  }
  return sum4(acc);
}

// The forward gives each row eight lanes (D / 8 values each; the dot products
// combine with three cross-lane adds), so 32 rows per workgroup: twice the
// workgroups, and waves, of four lanes per row on the same batch, which the
// tile loop's LDS broadcast reads need to hide their latency.  K / V tiles are
// double-buffered: each thread loads its share of the next tile into registers
// before the current tile's arithmetic and stores it to the other LDS buffer
// after, so one barrier per tile remains and the global loads' latency hides
// behind the arithmetic (staged synchronously, it was paid once per tile).
constexpr int kFwdLanes = 8;
constexpr int kFwdRows = kThreads / kFwdLanes;

template <int D>
__global__ __launch_bounds__(kThreads) void fwd_f32_kernel(const F32Args a) {
  constexpr int EPL = D / kFwdLanes;
  static_assert(EPL % 4 == 0, "whole float4 per lane");
  constexpr int V4 = D / 4;
  constexpr int kVecs = kTile * V4 / kThreads;  // float4 of K (and of V) per thread per tile
  static_assert(kVecs * kThreads == kTile * V4, "a tile divides evenly over the threads");
  __shared__ __attribute__((aligned(16))) float sK[2][kTile * D];
  __shared__ __attribute__((aligned(16))) float sV[2][kTile * D];
  const int h = blockIdx.x % a.Hq;
  const int s = blockIdx.x / a.Hq;
  const int tile = a.num_tiles - 1 - (int)blockIdx.y;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = tile * kFwdRows;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;
  const int sub = threadIdx.x % kFwdLanes;
  const int qpos = m0 + threadIdx.x / kFwdLanes;
  const bool valid = qpos < g.nq;
  const int kend = kend_of(g.p, qpos);
  const int wg_kend = max(g.p, min(m0 + kFwdRows, g.nq));

  float qv[EPL], acc[EPL];
  {
    const float* qrow = a.q + (int64_t)(g.start + qpos) * a.q_st + (int64_t)h * a.q_sh + sub * EPL;
#pragma unroll
    for (int e = 0; e < EPL; e += 4) {
      const f32x4 t = valid ? *(const f32x4*)&qrow[e] : f32x4{0.f, 0.f, 0.f, 0.f};
      qv[e] = t[0]; qv[e + 1] = t[1]; qv[e + 2] = t[2]; qv[e + 3] = t[3];
    }
  }
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  const float* kb = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const float* vb = a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh;

  // this thread's share of a tile: float4 column c of row `row`, kVecs of them
  f32x4 nk[kVecs], nv[kVecs];
  auto fetch = [&](int k0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kVecs; ++i) {
      const int idx = (int)threadIdx.x + i * kThreads, row = idx / V4, c = idx % V4;
      const bool in = k0 + row < g.n;
      nk[i] = in ? *(const f32x4*)&kb[(int64_t)(k0 + row) * a.k_st + 4 * c] : f32x4{0.f, 0.f, 0.f, 0.f};
      nv[i] = in ? *(const f32x4*)&vb[(int64_t)(k0 + row) * a.v_st + 4 * c] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto put = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kVecs; ++i) {
      const int idx = (int)threadIdx.x + i * kThreads, row = idx / V4, c = idx % V4;
      *(f32x4*)&sK[buf][row * D + 4 * c] = nk[i];
      *(f32x4*)&sV[buf][row * D + 4 * c] = nv[i];
    }
  };
  // The tile's arithmetic; false: no allowed key yet (only for rows with kend <= k0).
  auto tile_step = [&](int k0, const float* tK, const float* tV) __attribute__((always_inline)) {
    float sc[kTile];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      float x = 0.f;
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const f32x4 t = *(const f32x4*)&tK[j * D + sub * EPL + e];
        x = __builtin_fmaf(qv[e], t[0], x);
        x = __builtin_fmaf(qv[e + 1], t[1], x);
        x = __builtin_fmaf(qv[e + 2], t[2], x);
        x = __builtin_fmaf(qv[e + 3], t[3], x);
      }
      x += __shfl_xor(x, 1, 64);
      x += __shfl_xor(x, 2, 64);
      x += __shfl_xor(x, 4, 64);
      if (k0 + j >= kend) x = -INFINITY;
      sc[j] = x;
      mx = fmaxf(mx, x);
    }
    const float m_new = fmaxf(m_run, mx);
    if (m_new == -INFINITY) return;
    const float alpha = fast_exp2((m_run - m_new) * a.scale_log2);
    const float mb = m_new * a.scale_log2;
    l_run *= alpha;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int j = 0; j < kTile; ++j) {
      const float pr = fast_exp2(__builtin_fmaf(sc[j], a.scale_log2, -mb));
      l_run += pr;
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const f32x4 t = *(const f32x4*)&tV[j * D + sub * EPL + e];
        acc[e] = __builtin_fmaf(pr, t[0], acc[e]);
        acc[e + 1] = __builtin_fmaf(pr, t[1], acc[e + 1]);
        acc[e + 2] = __builtin_fmaf(pr, t[2], acc[e + 2]);
        acc[e + 3] = __builtin_fmaf(pr, t[3], acc[e + 3]);
      }
    }
    m_run = m_new;
  };

  if (wg_kend > 0) {
    fetch(0);
    put(0);
  }
  __syncthreads();
  for (int k0 = 0, buf = 0; k0 < wg_kend; k0 += kTile, buf ^= 1) {
    const bool more = k0 + kTile < wg_kend;
    if (more) fetch(k0 + kTile);  // in flight during this tile's arithmetic
    tile_step(k0, sK[buf], sV[buf]);
    // The other buffer's last readers finished this tile's predecessor before the
    // barrier that ended it; this tile's readers finish before the next barrier.
    if (more) put(buf ^ 1);
    __syncthreads();
  }
  if (!valid) return;
  const float inv = 1.f / l_run;
  float* orow = a.o + (int64_t)(g.start + qpos) * a.o_st + (int64_t)h * a.o_sh + sub * EPL;
#pragma unroll
  for (int e = 0; e < EPL; e += 4)
    *(f32x4*)&orow[e] = f32x4{acc[e] * inv, acc[e + 1] * inv, acc[e + 2] * inv, acc[e + 3] * inv};
  if (sub == 0 && a.lse != nullptr)
    a.lse[(int64_t)h * a.lse_sh + g.start + qpos] = m_run * a.scale + logf(l_run);
}

template <int D>
__global__ __launch_bounds__(256) void delta_f32_kernel(const F32Args a) {
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 2);
  const int sub = threadIdx.x & 3;
  const bool valid = row < (int64_t)a.T * a.Hq;
  const int t = valid ? (int)(row / a.Hq) : 0;
  const int h = valid ? (int)(row % a.Hq) : 0;
  float acc = 0.f;
  if (valid) {
    const float* orow = a.out + (int64_t)t * a.o_st + (int64_t)h * a.o_sh + sub * (D / 4);
    const float* drow = a.dout + (int64_t)t * a.do_st + (int64_t)h * a.do_sh + sub * (D / 4);
    for (int e = 0; e < D / 4; ++e) acc = __builtin_fmaf(orow[e], drow[e], acc);
  }
  acc = sum4(acc);
  if (valid && sub == 0) a.delta[(int64_t)h * a.T + t] = acc;
}

template <int D>
__global__ __launch_bounds__(kThreads) void dq_f32_kernel(const F32Args a) {
  constexpr int EPL = D / 4;
  __shared__ __attribute__((aligned(16))) float sK[kTile * D];
  __shared__ __attribute__((aligned(16))) float sV[kTile * D];
  const int h = blockIdx.x % a.Hq;
  const int s = blockIdx.x / a.Hq;
  const int tile = a.num_tiles - 1 - (int)blockIdx.y;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = tile * kRowsPerBlock;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;
  const int sub = threadIdx.x & 3;
  const int qpos = m0 + (threadIdx.x >> 2);
  const bool valid = qpos < g.nq;
  const int kend = kend_of(g.p, qpos);
  const int wg_kend = max(g.p, min(m0 + kRowsPerBlock, g.nq));

  float qv[EPL], dov[EPL], acc[EPL];
  load_row<D>(qv, a.q + (int64_t)(g.start + qpos) * a.q_st + (int64_t)h * a.q_sh, sub, valid);
  load_row<D>(dov, a.dout + (int64_t)(g.start + qpos) * a.do_st + (int64_t)h * a.do_sh, sub, valid);
#pragma unroll
  for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
  const float lse2 = valid ? a.olse[(int64_t)h * a.lse_sh + g.start + qpos] * kLog2e : 0.f;
  const float dlt = valid ? a.delta[(int64_t)h * a.T + g.start + qpos] : 0.f;
  const float* kb = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const float* vb = a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh;

  for (int k0 = 0; k0 < wg_kend; k0 += kTile) {
    __syncthreads();
    stage<D>(sK, kb, a.k_st, k0, g.n);
    stage<D>(sV, vb, a.v_st, k0, g.n);
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < kTile; ++j) {
      const float sc = dot_tile<D>(qv, &sK[j * D], sub);
      const float dp = dot_tile<D>(dov, &sV[j * D], sub);
      float pr = fast_exp2(__builtin_fmaf(sc, a.scale_log2, -lse2));
      if (!valid || k0 + j >= kend) pr = 0.f;
      const float ds = pr * (dp - dlt);
#pragma unroll
      for (int e = 0; e < EPL; e += 4) {
        const f32x4 t = *(const f32x4*)&sK[j * D + sub * EPL + e];
        acc[e] = __builtin_fmaf(ds, t[0], acc[e]);
        acc[e + 1] = __builtin_fmaf(ds, t[1], acc[e + 1]);
        acc[e + 2] = __builtin_fmaf(ds, t[2], acc[e + 2]);
        acc[e + 3] = __builtin_fmaf(ds, t[3], acc[e + 3]);
      }
    }
  }
  if (!valid) return;
  float* drow = a.dq + (int64_t)(g.start + qpos) * a.dq_st + (int64_t)h * a.dq_sh + sub * EPL;
#pragma unroll
  for (int e = 0; e < EPL; e += 4)
    *(f32x4*)&drow[e] = f32x4{acc[e] * a.scale, acc[e + 1] * a.scale, acc[e + 2] * a.scale, acc[e + 3] * a.scale};
}

template <int D>
__global__ __launch_bounds__(kThreads) void dkdv_f32_kernel(const F32Args a) {
  constexpr int EPL = D / 4;
  __shared__ __attribute__((aligned(16))) float sQ[kTile * D];
  __shared__ __attribute__((aligned(16))) float sO[kTile * D];
  __shared__ float sL[kTile];
  __shared__ float sD[kTile];
  const int hk = blockIdx.x % a.Hkv;
  const int s = blockIdx.x / a.Hkv;
  const int tile = blockIdx.y;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int k0 = tile * kRowsPerBlock;
  if (k0 >= g.n) return;
  const int sub = threadIdx.x & 3;
  const int kpos = k0 + (threadIdx.x >> 2);
  const bool valid = kpos < g.n;
  const int qs = qstart_of(g.p, kpos);
  const int q_begin = qstart_of(g.p, k0);

  float kv[EPL], vv[EPL], dka[EPL], dva[EPL];
  load_row<D>(kv, a.k + (int64_t)(g.start + kpos) * a.k_st + (int64_t)hk * a.k_sh, sub, valid);
  load_row<D>(vv, a.v + (int64_t)(g.start + kpos) * a.v_st + (int64_t)hk * a.v_sh, sub, valid);
#pragma unroll
  for (int e = 0; e < EPL; ++e) { dka[e] = 0.f; dva[e] = 0.f; }

  for (int hh = 0; hh < a.group; ++hh) {
    const int h = hk * a.group + hh;
    const float* qb = a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh;
    const float* ob = a.dout + (int64_t)g.start * a.do_st + (int64_t)h * a.do_sh;
    for (int q0 = q_begin; q0 < g.nq; q0 += kTile) {
      __syncthreads();
      stage<D>(sQ, qb, a.q_st, q0, g.nq);
      stage<D>(sO, ob, a.do_st, q0, g.nq);
      if (threadIdx.x < kTile) {
        const int qr = q0 + threadIdx.x;
        const bool ok = qr < g.nq;
        sL[threadIdx.x] = ok ? a.olse[(int64_t)h * a.lse_sh + g.start + qr] * kLog2e : 0.f;
        sD[threadIdx.x] = ok ? a.delta[(int64_t)h * a.T + g.start + qr] : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int i = 0; i < kTile; ++i) {
        const int qp = q0 + i;
        const float sc = dot_tile<D>(kv, &sQ[i * D], sub);
        const float dp = dot_tile<D>(vv, &sO[i * D], sub);
        float pr = fast_exp2(__builtin_fmaf(sc, a.scale_log2, -sL[i]));
        if (!valid || qp < qs || qp >= g.nq) pr = 0.f;
        const float ds = pr * (dp - sD[i]);
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          const f32x4 tq = *(const f32x4*)&sQ[i * D + sub * EPL + e];
          const f32x4 to = *(const f32x4*)&sO[i * D + sub * EPL + e];
          dva[e] = __builtin_fmaf(pr, to[0], dva[e]);
          dva[e + 1] = __builtin_fmaf(pr, to[1], dva[e + 1]);
          dva[e + 2] = __builtin_fmaf(pr, to[2], dva[e + 2]);
          dva[e + 3] = __builtin_fmaf(pr, to[3], dva[e + 3]);
          dka[e] = __builtin_fmaf(ds, tq[0], dka[e]);
          dka[e + 1] = __builtin_fmaf(ds, tq[1], dka[e + 1]);
          dka[e + 2] = __builtin_fmaf(ds, tq[2], dka[e + 2]);
          dka[e + 3] = __builtin_fmaf(ds, tq[3], dka[e + 3]);
        }
      }
    }
  }
  if (!valid) return;
  float* krow = a.dk + (int64_t)(g.start + kpos) * a.dk_st + (int64_t)hk * a.dk_sh + sub * EPL;
  float* vrow = a.dv + (int64_t)(g.start + kpos) * a.dv_st + (int64_t)hk * a.dv_sh + sub * EPL;
#pragma unroll
  for (int e = 0; e < EPL; e += 4) {
    *(f32x4*)&krow[e] = f32x4{dka[e] * a.scale, dka[e + 1] * a.scale, dka[e + 2] * a.scale, dka[e + 3] * a.scale};
    *(f32x4*)&vrow[e] = f32x4{dva[e], dva[e + 1], dva[e + 2], dva[e + 3]};
  }
}

F32Args common_args(int T, int Hq, int Hkv, int total_seqlen, int is_causal, float scale,
                    const int32_t* prefix_lens, const int32_t* cu_seqlens) {
  F32Args a = {};
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.group = Hq / Hkv;
  a.total_seqlen = total_seqlen;
  a.is_causal = is_causal;
  a.scale = scale;
  a.scale_log2 = scale * kLog2e;
  a.prefix_lens = prefix_lens;
  a.cu_seqlens = cu_seqlens;
  return a;
}

template <int D>
hipError_t launch_fwd(const MimirPrefixLMFwdParams& p, hipStream_t stream) {
  F32Args a = common_args(p.total_tokens, p.num_q_heads, p.num_kv_heads, p.total_seqlen, p.is_causal,
                          p.softmax_scale, p.prefix_lens, p.cu_seqlens);
  a.q = (const float*)p.q; a.k = (const float*)p.k; a.v = (const float*)p.v;
  a.o = (float*)p.out; a.lse = p.lse;
  a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.k_st = p.k_stride_token; a.k_sh = p.k_stride_head;
  a.v_st = p.v_stride_token; a.v_sh = p.v_stride_head;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.lse_sh = p.lse_stride_head;
  a.num_tiles = (p.max_seqlen_all + kFwdRows - 1) / kFwdRows;
  if (a.num_tiles == 0 || p.numseqs == 0) return hipSuccess;
  hipLaunchKernelGGL(fwd_f32_kernel<D>, dim3(p.num_q_heads * p.numseqs, a.num_tiles), dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_bwd(const MimirPrefixLMBwdParams& p, hipStream_t stream, int stages) {
  F32Args a = common_args(p.total_tokens, p.num_q_heads, p.num_kv_heads, p.total_seqlen, p.is_causal,
                          p.softmax_scale, p.prefix_lens, p.cu_seqlens);
  a.q = (const float*)p.q; a.k = (const float*)p.k; a.v = (const float*)p.v;
  a.out = (const float*)p.out; a.dout = (const float*)p.dout; a.olse = p.lse;
  a.dq = (float*)p.dq; a.dk = (float*)p.dk; a.dv = (float*)p.dv;
  a.delta = (float*)p.workspace;
  a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.k_st = p.k_stride_token; a.k_sh = p.k_stride_head;
  a.v_st = p.v_stride_token; a.v_sh = p.v_stride_head;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.do_st = p.dout_stride_token; a.do_sh = p.dout_stride_head;
  a.dq_st = p.dq_stride_token; a.dq_sh = p.dq_stride_head;
  a.dk_st = p.dk_stride_token; a.dk_sh = p.dk_stride_head;
  a.dv_st = p.dv_stride_token; a.dv_sh = p.dv_stride_head;
  a.lse_sh = p.lse_stride_head;
  a.num_tiles = (p.max_seqlen_all + kRowsPerBlock - 1) / kRowsPerBlock;
  const int64_t rows = (int64_t)p.total_tokens * p.num_q_heads;
  if (rows > 0 && (stages & MIMIR_BWD_STAGE_DELTA))
    hipLaunchKernelGGL(delta_f32_kernel<D>, dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                       dim3(256), 0, stream, a);
  if (a.num_tiles > 0 && p.numseqs > 0) {
    if (stages & MIMIR_BWD_STAGE_DQ)
      hipLaunchKernelGGL(dq_f32_kernel<D>, dim3(p.num_q_heads * p.numseqs, a.num_tiles), dim3(kThreads), 0,
                         stream, a);
    if (stages & MIMIR_BWD_STAGE_DKDV)
      hipLaunchKernelGGL(dkdv_f32_kernel<D>, dim3(p.num_kv_heads * p.numseqs, a.num_tiles), dim3(kThreads), 0,
                         stream, a);
  }
  return hipGetLastError();
}

}  // namespace

bool mimir_f32_head_dim_supported(int d) { return d == 32 || d == 64 || d == 96 || d == 128; }

hipError_t mimir_launch_fwd_f32(const MimirPrefixLMFwdParams& p, hipStream_t stream) {
  switch (p.head_dim) {
    case 32: return launch_fwd<32>(p, stream);
    case 64: return launch_fwd<64>(p, stream);
    case 96: return launch_fwd<96>(p, stream);
    case 128: return launch_fwd<128>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t mimir_launch_bwd_f32(const MimirPrefixLMBwdParams& p, hipStream_t stream, int stages) {
  switch (p.head_dim) {
    case 32: return launch_bwd<32>(p, stream, stages);
    case 64: return launch_bwd<64>(p, stream, stages);
    case 96: return launch_bwd<96>(p, stream, stages);
    case 128: return launch_bwd<128>(p, stream, stages);
    default: return hipErrorInvalidValue;
  }
}
