// Attention against a static KV cache (inference), bf16, for gfx950 (MI355X).
//
// Reference: src/mimir/model/layers.py:134-167 (_attention_with_cache).  The
// new keys / values go into the cache at positions cache_lengths[b] + i, then
// every query row attends the cache keys j < kv_len = cache_lengths[b] + S
// (and j <= cache_lengths[b] + i when causal).  The reference materializes the
// repeated K/V heads and a [B, S, max_kv_len] mask for SDPA; here:
//
//   cache_append_kernel   the scatter of k_new / v_new into the cache rows (it
//                         also clears the split arrival counters)
//   cache_attn_kernel     one workgroup per (batch row, kv head, 128 query rows,
//                         key split): the G query heads of a kv head share its
//                         K / V tiles (rows are (token, head) pairs, token-major),
//                         64-key tiles stream through two LDS stages, S^T = K Q^T
//                         and O^T += V^T P^T on bf16 MFMA with an online softmax
//                         (the forward kernel's arithmetic).  With several
//                         splits, each publishes its partial (max, sum, O) rows
//                         and the last to arrive merges them into the output.
//
// Decode (S = 1) has only G rows per kv head, so each batch row's key range is
// split evenly over enough workgroups to cover the chip (flash-decoding); the
// kernel is then bound by the HBM read of the cache.  Prefill with a long S
// fills the row tiles and runs on the MFMA like the forward kernel.
#include "prefixlm_common.h"

namespace mimir {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = kWaves * 32;  // query rows per workgroup
constexpr int kKeys = 64;           // keys per tile
constexpr int kMaxSplits = 64;      // key splits per row tile

struct CacheArgs {
  const bf16_t* q;
  const bf16_t* kn;
  const bf16_t* vn;
  bf16_t* ck;
  bf16_t* cv;
  bf16_t* out;
  const void* cache_lengths;  // int32 or int64 (idx64)
  const void* batch_indices;  // int32 or int64, or null
  int idx64;
  int64_t q_sb, q_st, q_sh, kn_sb, kn_st, kn_sh, vn_sb, vn_st, vn_sh;
  int64_t ck_sb, ck_st, ck_sh, cv_sb, cv_st, cv_sh, o_sb, o_st, o_sh;
  int B, S, L, rows, Hkv, G, causal, D;
  int n_rt;        // row tiles per (batch row, kv head)
  int splits;      // key splits per row tile (each batch row's key tiles spread evenly over them)
  float scale_log2;
  float* part_o;   // [unit, kRows, D] unnormalized O of each split (splits > 1)
  float* part_ml;  // [unit, kRows, 2]: running max (exp2 domain) and sum
  int* counters;   // [B * Hkv * n_rt] split arrivals per row tile (splits > 1), cleared by the append kernel
  int n_counters;
};

__device__ __forceinline__ int64_t load_index(const void* p, int i, int idx64) {
  return idx64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}
__device__ __forceinline__ int64_t cache_row(const CacheArgs& a, int b) {
  return a.batch_indices != nullptr ? load_index(a.batch_indices, b, a.idx64) : b;
}
// cache_lengths[b] clamped to [0, L]
__device__ __forceinline__ int cache_len_of(const CacheArgs& a, int b) {
  const int64_t c = load_index(a.cache_lengths, b, a.idx64);
  return c < 0 ? 0 : (c > a.L ? a.L : (int)c);
}

// k_new / v_new [b, i, h] -> cache [row(b), cache_lengths[b] + i, h]; 16 bytes per thread.
__global__ __launch_bounds__(256) void cache_append_kernel(const CacheArgs a) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < a.n_counters; i += gridDim.x * 256) a.counters[i] = 0;
  const int chunks = a.D / 8;
  const int64_t total = (int64_t)a.B * a.S * a.Hkv * chunks;
  for (int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (int64_t)gridDim.x * 256) {
    const int c = (int)(idx % chunks);
    int64_t t = idx / chunks;
    const int h = (int)(t % a.Hkv);
    t /= a.Hkv;
    const int i = (int)(t % a.S);
    const int b = (int)(t / a.S);
    const int64_t pos = load_index(a.cache_lengths, b, a.idx64) + i;
    const int64_t r = cache_row(a, b);
    if (pos < 0 || pos >= a.L || r < 0 || r >= a.rows) continue;  // outside the cache: dropped
    *(bf16x8*)&a.ck[r * a.ck_sb + (int64_t)pos * a.ck_st + (int64_t)h * a.ck_sh + c * 8] =
        *(const bf16x8*)&a.kn[(int64_t)b * a.kn_sb + (int64_t)i * a.kn_st + (int64_t)h * a.kn_sh + c * 8];
    *(bf16x8*)&a.cv[r * a.cv_sb + (int64_t)pos * a.cv_st + (int64_t)h * a.cv_sh + c * 8] =
        *(const bf16x8*)&a.vn[(int64_t)b * a.vn_sb + (int64_t)i * a.vn_st + (int64_t)h * a.vn_sh + c * 8];
  }
}

constexpr int kDevScope = 16;  // buffer cache policy: coherent at device scope

// Output rows [0, rt_rows) of row tile rt of (batch row b, kv head hk): the
// merge of the partial (max in the exp2 domain, sum, unnormalized O) rows that
// the n_valid splits of `group` published at slots (group * splits + c) * kRows
// + row.  out = sum_c O_c 2^(m_c - M) / sum_c l_c 2^(m_c - M); one wave per row
// (waves of a kWaves-wave workgroup), D / 64 columns per lane.  The splits are
// merged online in chunks of eight whose loads ((max, sum) and the lane's O
// columns) are all issued before any is used, so a chunk costs one memory
// round trip.  The loads are device-coherent: the caller has seen every split
// arrive.
template <int D>
__device__ void merge_split_rows(const CacheArgs& a, const __amdgpu_buffer_rsrc_t ro,
                                 const __amdgpu_buffer_rsrc_t rml, int group, int n_valid, int b, int hk, int rt,
                                 int rt_rows, int wave, int lane) {
  const uint32_t unit0 = (uint32_t)group * a.splits;
  constexpr int cpl = D / 64;
  constexpr int kChunk = 8;
  for (int rr = wave; rr < rt_rows; rr += kWaves) {
    float M = -INFINITY, lsum = 0.f;
    float acc[cpl] = {};
    for (int c0 = 0; c0 < n_valid; c0 += kChunk) {
      f32x2 ml[kChunk];
      float ov[kChunk][cpl];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const uint32_t slot = (unit0 + min(c0 + i, n_valid - 1)) * kRows + rr;
        ml[i] = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rml, slot * 8, 0, kDevScope));
        const uint32_t off = (slot * D + lane * cpl) * 4;
        if constexpr (cpl == 2) {
          const f32x2 o = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(ro, off, 0, kDevScope));
          ov[i][0] = o[0];
          ov[i][1] = o[1];
        } else {
          ov[i][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ro, off, 0, kDevScope));
        }
      }
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        if (c0 + i >= n_valid) break;
        const float m = ml[i][0];
        if (m == -INFINITY) continue;  // no allowed key in this split
        const float m_new = fmaxf(M, m);
        const float alpha = M == -INFINITY ? 0.f : fast_exp2(M - m_new);  // rescale the running sums
        const float w = fast_exp2(m - m_new);
        lsum = lsum * alpha + ml[i][1] * w;
#pragma unroll
        for (int j = 0; j < cpl; ++j) acc[j] = acc[j] * alpha + ov[i][j] * w;
        M = m_new;
      }
    }
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const int row_g = rt * kRows + rr;
    const int ti_r = row_g / a.G;
    const int h_r = hk * a.G + (row_g - ti_r * a.G);
    bf16_t* orow = a.out + (int64_t)b * a.o_sb + (int64_t)ti_r * a.o_st + (int64_t)h_r * a.o_sh + lane * cpl;
#pragma unroll
    for (int i = 0; i < cpl; ++i) orow[i] = (bf16_t)(acc[i] * inv);
  }
}

template <int D>
__global__ __launch_bounds__(kThreads, 2) void cache_attn_kernel(const CacheArgs a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  using L = TileLayout<D>;
  __shared__ __attribute__((aligned(16))) bf16_t sK0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sK1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV1[L::kElems];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  int u = blockIdx.x;
  const int split = u % a.splits;
  u /= a.splits;
  const int rt = u % a.n_rt;
  u /= a.n_rt;
  const int hk = u % a.Hkv;
  const int b = u / a.Hkv;

  const int64_t crow = cache_row(a, b);
  const bool row_in_cache = crow >= 0 && crow < a.rows;
  const int clen = cache_len_of(a, b);
  const int kv = row_in_cache ? min(clen + a.S, a.L) : 0;  // keys of this batch row
  // This batch row's key tiles, spread evenly over the splits; n_valid splits
  // hold keys.  A row without keys (outside the cache) gets zeros from split 0.
  const int tiles_b = (kv + kKeys - 1) / kKeys;
  const int per = max(1, (tiles_b + a.splits - 1) / a.splits);
  const int n_valid = (tiles_b + per - 1) / per;
  if (split > 0 && split >= n_valid) return;
  const int k0 = split * per * kKeys;
  const int k1 = min(kv, k0 + per * kKeys);
  const int R = a.S * a.G;  // query rows (token-major (token, head) pairs)

  // This lane's row and its key limit.
  const int row = rt * kRows + wave * 32 + l32;
  const bool row_ok = row < R;
  const int ti = row_ok ? row / a.G : 0;
  const int h = hk * a.G + (row_ok ? row - ti * a.G : 0);
  const int kend_lane = row_ok ? (a.causal ? min(clen + ti + 1, kv) : kv) : 0;
  // Wave-wide bounds (rows are token-major, so the wave's last row has the largest limit).
  const int r0 = rt * kRows + wave * 32;
  const bool wave_active = r0 < R;
  const int r_last = min(r0 + 31, R - 1);
  const int w_kend_max = wave_active ? (a.causal ? min(clen + r_last / a.G + 1, kv) : kv) : 0;
  const int w_kend_min = wave_active ? (a.causal ? min(clen + r0 / a.G + 1, kv) : kv) : 0;
  // Workgroup range of key tiles inside this split.
  const int wg_r_last = min(rt * kRows + kRows - 1, R - 1);
  const int wg_kend = a.causal ? min(clen + wg_r_last / a.G + 1, kv) : kv;
  const int kt0 = k0 / kKeys;
  const int kt1 = (min(k1, wg_kend) + kKeys - 1) / kKeys;  // may be <= kt0: nothing to attend

  const bf16_t* kbase = a.ck + (row_in_cache ? crow : 0) * a.ck_sb + (int64_t)hk * a.ck_sh;
  const bf16_t* vbase = a.cv + (row_in_cache ? crow : 0) * a.cv_sb + (int64_t)hk * a.cv_sh;
  const TileLoader<D, kWaves> ldk(a.ck_st, wave, lane), ldv(a.cv_st, wave, lane);
  if (kt0 < kt1) {
    ldk.issue(kbase, kt0 * kKeys, kv, sK0);
    ldv.issue(vbase, kt0 * kKeys, kv, sV0);
  }

  // Q^T B-operand fragments: lane holds row `row`, d = 16*ks + 8*hi .. +7 (0 for rows >= R).
  bf16x8 qf[KS];
  {
    const bf16_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)ti * a.q_st + (int64_t)h * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = row_ok ? *(const bf16x8*)&qrow[16 * ks + 8 * hi] : bf16x8{};
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  auto compute = [&](int kt, const bf16_t* sK, const bf16_t* sV) {
    const int kb = kt * kKeys;
    if (!wave_active || kb >= w_kend_max) return;
    f32x16 st[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      st[mt] = f32x16{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8 kf = *(const bf16x8*)&sK[tl.op_base + mt * 32 * L::kRowElems + ks * 16];
        st[mt] = mfma32(kf, qf[ks], st[mt]);
      }
    }
    if (kb + kKeys > w_kend_min) {
      __asm__ volatile("");
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int kpos = kb + 32 * mt + 8 * (r >> 2) + 4 * hi + (r & 3);
          if (kpos >= kend_lane) st[mt][r] = -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[mt][r]);
    mx = xor32_max(mx);
    // Lazy rescaling, as in the forward kernel: the reference max moves only
    // when it grows by more than 2^8 in probability terms.
    const float m_cand = fmaxf(m_run, mx);
    const bool grow = (m_cand - m_run) * c2 > 8.f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? m_cand : m_run;
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      m_run = m_new;
    }
    const float mb = m_run == -INFINITY ? 0.f : m_run * c2;
    float lsum = 0.f;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float pr = fast_exp2(__builtin_fmaf(st[mt][r], c2, -mb));
        st[mt][r] = pr;
        lsum += pr;
      }
    l_run += lsum;
    bf16x8 pf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int mt = kk >> 1, s8 = (kk & 1) * 8;
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = st[mt][s8 + e];
      pf[kk] = to_bf16x8(t);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16_t* vp = &sV[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
        oacc[dt] = mfma32(cat8(lds_read_tr16(vp), lds_read_tr16(vp + L::kTrSecond)), pf[kk], oacc[dt]);
      }
  };

  for (int kt = kt0; kt < kt1; kt += 2) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < kt1) {
      ldk.issue(kbase, (kt + 1) * kKeys, kv, sK1);
      ldv.issue(vbase, (kt + 1) * kKeys, kv, sV1);
    }
    compute(kt, sK0, sV0);
    if (kt + 1 >= kt1) break;
    wait_vmem();
    __syncthreads();
    if (kt + 2 < kt1) {
      ldk.issue(kbase, (kt + 2) * kKeys, kv, sK0);
      ldv.issue(vbase, (kt + 2) * kKeys, kv, sV0);
    }
    compute(kt + 1, sK1, sV1);
  }

  const float l_tot = xor32_sum(l_run);
  if (n_valid <= 1) {
    if (!wave_active || !row_ok) return;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;  // no keys (row outside the cache): zeros
    bf16_t* orow = a.out + (int64_t)b * a.o_sb + (int64_t)ti * a.o_st + (int64_t)h * a.o_sh;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = oacc[dt][4 * rg + e] * inv;
        *(bf16x4*)&orow[32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(t, bf16x4);
      }
    return;
  }

  // Several splits hold keys of this row tile: publish this split's partial
  // rows -- unnormalized O, the max in the exp2 domain (-inf: no allowed key)
  // and the sum -- with device-coherent stores; the last split to arrive (per
  // row tile) reads them all back the same way and writes the merged rows.
  // The stores are complete before the arrival count, and the loads are issued
  // after it has returned, so no cache flush is needed.
  const int64_t units = (int64_t)gridDim.x;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.part_o, (uint32_t)(units * kRows * D * 4));
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(a.part_ml, (uint32_t)(units * kRows * 2 * 4));
  const int rt_rows = min(kRows, R - rt * kRows);
  if (wave_active) {
    const uint32_t slot = (uint32_t)blockIdx.x * kRows + wave * 32 + l32;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 t;
#pragma unroll
        for (int e = 0; e < 4; ++e) t[e] = oacc[dt][4 * rg + e];
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, t), ro,
                                               (slot * D + 32 * dt + 8 * rg + 4 * hi) * 4, 0, kDevScope);
      }
    if (hi == 0) {
      const float m2 = m_run == -INFINITY ? -INFINITY : m_run * c2;
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, f32x2{m2, l_tot}), rml, slot * 8, 0,
                                            kDevScope);
    }
  }
  __asm__ volatile("" ::: "memory");
  wait_vmem();  // the partial rows are stored
  __shared__ int last;
  __syncthreads();
  const int group = blockIdx.x / a.splits;  // (batch row, kv head, row tile)
  if (tid == 0)
    last = __hip_atomic_fetch_add(&a.counters[group], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_valid - 1;
  __syncthreads();
  if (!last) return;
  merge_split_rows<D>(a, ro, rml, group, n_valid, b, hk, rt, rt_rows, wave, lane);
}

// ---------------------------------------------------------------------------
// Decode: at most 32 query rows per kv head (S * G <= 32, e.g. S = 1).  The
// rows fit one wave, so instead of sharing 64-key tiles behind workgroup
// barriers, each of the four waves streams its own 32-key tiles of the split
// (tiles t0 + w, t0 + w + 4, ...) through two LDS stages of its own and waits
// only for its own copies: four independent copy pipelines per workgroup, one
// workgroup per CU.  The waves' partial rows are merged through LDS, and the
// splits of a batch row through memory as in cache_attn_kernel.
// ---------------------------------------------------------------------------
constexpr int kDecKeys = 32;  // keys per wave tile
constexpr int kDecRows = 32;  // query rows of the decode kernel (one wave's columns)

template <int D>
struct DecTile {
  using L = TileLayout<D>;
  static constexpr int kUnits = kDecKeys * L::kRowUnits;  // 16-byte units of a 32-row tile
  static constexpr int kInst = (kUnits + 63) / 64;        // wave copy instructions per tile
  static constexpr int kElems = kInst * 512;              // bf16 elements incl. the last instruction's tail
};

// s_waitcnt vmcnt(N) for N < 64 (expcnt and lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt_wide() {
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

template <int D>
__device__ __forceinline__ void cache_decode_body(const CacheArgs& a) {
  constexpr int DT = D / 32;
  constexpr int KS = D / 16;
  using L = TileLayout<D>;
  using T = DecTile<D>;
  // two stages of (K, V) per wave; each stage array holds the four waves' tiles
  __shared__ __attribute__((aligned(16))) bf16_t sK0[kWaves * T::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[kWaves * T::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sK1[kWaves * T::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV1[kWaves * T::kElems];
  __shared__ __attribute__((aligned(16))) float sMl[kWaves][kDecRows][2];  // per wave and row: max (exp2), sum
  static_assert(2 * kDecRows * D * 4 <= kWaves * T::kElems * 2, "two waves' partial O fit one stage array");
  __shared__ int last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  const int split = blockIdx.x % a.splits;
  const int group = blockIdx.x / a.splits;  // (batch row, kv head); one row tile
  const int hk = group % a.Hkv;
  const int b = group / a.Hkv;
  const int64_t crow = cache_row(a, b);
  const bool row_in_cache = crow >= 0 && crow < a.rows;
  const int clen = cache_len_of(a, b);
  const int kv = row_in_cache ? min(clen + a.S, a.L) : 0;
  // This batch row's 32-key tiles, spread evenly over the splits.
  const int tiles_b = (kv + kDecKeys - 1) / kDecKeys;
  const int per = max(1, (tiles_b + a.splits - 1) / a.splits);
  const int n_valid = (tiles_b + per - 1) / per;
  if (split > 0 && split >= n_valid) return;
  const int t0 = split * per;
  const int R = a.S * a.G;  // <= kDecRows
  const int row = l32;
  const bool row_ok = row < R;
  const int ti = row_ok ? row / a.G : 0;
  const int h = hk * a.G + (row_ok ? row - ti * a.G : 0);
  const int kend_lane = row_ok ? (a.causal ? min(clen + ti + 1, kv) : kv) : 0;
  const int kend_max = a.causal ? min(clen + (R - 1) / a.G + 1, kv) : kv;
  const int kend_min = a.causal ? min(clen + 1, kv) : kv;
  const int t_end = min(min(tiles_b, t0 + per), (kend_max + kDecKeys - 1) / kDecKeys);
  const int n_my = t0 + wave < t_end ? (t_end - t0 - wave + kWaves - 1) / kWaves : 0;  // this wave's tiles

  // Q^T B-operand fragments first (their loads are older than every tile copy).
  bf16x8 qf[KS];
  {
    const bf16_t* qrow = a.q + (int64_t)b * a.q_sb + (int64_t)ti * a.q_st + (int64_t)h * a.q_sh;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = row_ok ? *(const bf16x8*)&qrow[16 * ks + 8 * hi] : bf16x8{};
  }

  // This wave's copies of one 32-key tile: instruction i writes units
  // [64 i, 64 i + 64) of the wave's region; units past the 32 rows read zeros.
  const bf16_t* kbase = a.ck + (row_in_cache ? crow : 0) * a.ck_sb + (int64_t)hk * a.ck_sh;
  const bf16_t* vbase = a.cv + (row_in_cache ? crow : 0) * a.cv_sb + (int64_t)hk * a.cv_sh;
  uint32_t voffk[T::kInst], voffv[T::kInst];
#pragma unroll
  for (int i = 0; i < T::kInst; ++i) {
    const int u = i * 64 + lane;
    const int prow = u / L::kRowUnits;
    const int c = u - prow * L::kRowUnits;
    const int k = L::unperm(prow);
    const bool ok = c < L::kUnits && k < kDecKeys;
    voffk[i] = ok ? (uint32_t)((k * a.ck_st + c * 8) * 2) : 0x80000000u;
    voffv[i] = ok ? (uint32_t)((k * a.cv_st + c * 8) * 2) : 0x80000000u;
  }
  auto issue = [&](int t, bf16_t* tk, bf16_t* tv) {
    const int key0 = t * kDecKeys;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kbase + (int64_t)key0 * a.ck_st, rows_bytes(kv - key0, a.ck_st, D));
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vbase + (int64_t)key0 * a.cv_st, rows_bytes(kv - key0, a.cv_st, D));
#pragma unroll
    for (int i = 0; i < T::kInst; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(tk + i * 512), 16,
                                               voffk[i], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < T::kInst; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(tv + i * 512), 16,
                                               voffv[i], 0, 0, 0);
  };
  bf16_t* const mk0 = sK0 + wave * T::kElems;
  bf16_t* const mv0 = sV0 + wave * T::kElems;
  bf16_t* const mk1 = sK1 + wave * T::kElems;
  bf16_t* const mv1 = sV1 + wave * T::kElems;
  if (n_my > 0) issue(t0 + wave, mk0, mv0);
  if (n_my > 1) issue(t0 + wave + kWaves, mk1, mv1);

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c2 = a.scale_log2;
  const TileLanes<D> tl(lane);

  auto compute = [&](int t, const bf16_t* sK, const bf16_t* sV) {
    const int kb = t * kDecKeys;
    f32x16 st = f32x16{};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st = mfma32(*(const bf16x8*)&sK[tl.op_base + ks * 16], qf[ks], st);
    if (kb + kDecKeys > kend_min) {
      __asm__ volatile("");
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kpos = kb + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (kpos >= kend_lane) st[r] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, st[r]);
    mx = xor32_max(mx);
    // Lazy rescaling, as in the forward kernel.
    const float m_cand = fmaxf(m_run, mx);
    const bool grow = (m_cand - m_run) * c2 > 8.f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float m_new = grow ? m_cand : m_run;
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2((m_run - m_new) * c2);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      m_run = m_new;
    }
    const float mb = m_run == -INFINITY ? 0.f : m_run * c2;
    float lsum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr = fast_exp2(__builtin_fmaf(st[r], c2, -mb));
      st[r] = pr;
      lsum += pr;
    }
    l_run += lsum;
    bf16x8 pf[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f32x8 tv;
#pragma unroll
      for (int e = 0; e < 8; ++e) tv[e] = st[8 * kk + e];
      pf[kk] = to_bf16x8(tv);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const bf16_t* vp = &sV[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
        oacc[dt] = mfma32(cat8(lds_read_tr16(vp), lds_read_tr16(vp + L::kTrSecond)), pf[kk], oacc[dt]);
      }
  };

  // Each wave waits only for its own copies: tile i has landed once at most the
  // copies of tile i + 1 are outstanding.
  for (int i = 0; i < n_my; i += 2) {
    if (i + 1 < n_my)
      wait_vmcnt_wide<2 * T::kInst>();
    else
      wait_vmcnt_wide<0>();
    compute(t0 + wave + kWaves * i, mk0, mv0);
    if (i + 2 < n_my) {
      wait_lds();  // this wave's reads of the stage are done before it is refilled
      issue(t0 + wave + kWaves * (i + 2), mk0, mv0);
    }
    if (i + 1 >= n_my) break;
    if (i + 2 < n_my)
      wait_vmcnt_wide<2 * T::kInst>();
    else
      wait_vmcnt_wide<0>();
    compute(t0 + wave + kWaves * (i + 1), mk1, mv1);
    if (i + 3 < n_my) {
      wait_lds();
      issue(t0 + wave + kWaves * (i + 3), mk1, mv1);
    }
  }

  // Merge the four waves' partial rows through LDS (the stages are free once
  // every wave is past its tile loop): O of waves 0-1 in sK0, of waves 2-3 in sV0.
  __syncthreads();
  {
    float* po = (float*)(wave < 2 ? sK0 : sV0) + (wave & 1) * kDecRows * D + l32 * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 tv;
#pragma unroll
        for (int e = 0; e < 4; ++e) tv[e] = oacc[dt][4 * rg + e];
        *(f32x4*)&po[32 * dt + 8 * rg + 4 * hi] = tv;
      }
    const float l_tot = xor32_sum(l_run);
    if (hi == 0) {
      sMl[wave][l32][0] = m_run == -INFINITY ? -INFINITY : m_run * c2;
      sMl[wave][l32][1] = l_tot;
    }
  }
  __syncthreads();
  constexpr int cpl = D / 64;
  const int64_t units = (int64_t)gridDim.x;
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.part_o, (uint32_t)(units * kRows * D * 4));
  const __amdgpu_buffer_rsrc_t rml = make_rsrc(a.part_ml, (uint32_t)(units * kRows * 2 * 4));
  for (int rr = wave; rr < R; rr += kWaves) {  // one wave per row, D / 64 columns per lane
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sMl[w][rr][0]);
    float lsum = 0.f;
    float acc[cpl] = {};
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float m = sMl[w][rr][0];
        const float wt = m == -INFINITY ? 0.f : fast_exp2(m - M);
        lsum += sMl[w][rr][1] * wt;
        const float* po = (const float*)(w < 2 ? sK0 : sV0) + (w & 1) * kDecRows * D + rr * D + lane * cpl;
#pragma unroll
        for (int j = 0; j < cpl; ++j) acc[j] += po[j] * wt;
      }
    }
    if (n_valid <= 1) {
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;  // no keys (row outside the cache): zeros
      const int ti_r = rr / a.G;
      const int h_r = hk * a.G + (rr - ti_r * a.G);
      bf16_t* orow = a.out + (int64_t)b * a.o_sb + (int64_t)ti_r * a.o_st + (int64_t)h_r * a.o_sh + lane * cpl;
#pragma unroll
      for (int j = 0; j < cpl; ++j) orow[j] = (bf16_t)(acc[j] * inv);
    } else {
      // this split's partial row, published with device-coherent stores
      const uint32_t slot = (uint32_t)blockIdx.x * kRows + rr;
      if constexpr (cpl == 2)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, f32x2{acc[0], acc[1]}), ro,
                                              (slot * D + lane * 2) * 4, 0, kDevScope);
      else
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, acc[0]), ro, (slot * D + lane) * 4, 0,
                                              kDevScope);
      if (lane == 0)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, f32x2{M, lsum}), rml, slot * 8, 0,
                                              kDevScope);
    }
  }
  if (n_valid <= 1) return;
  __asm__ volatile("" ::: "memory");
  wait_vmem();  // the partial rows are stored
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(&a.counters[group], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n_valid - 1;
  __syncthreads();
  if (!last) return;
  merge_split_rows<D>(a, ro, rml, group, n_valid, b, hk, 0, R, wave, lane);
}

// One kernel per head_dim, by name: two instantiations of one kernel template
// launched from the two branches below lost one host stub in this toolchain.
__global__ __launch_bounds__(kThreads, 1) void cache_decode_d128_kernel(const CacheArgs a) {
  cache_decode_body<128>(a);
}
__global__ __launch_bounds__(kThreads, 1) void cache_decode_d64_kernel(const CacheArgs a) {
  cache_decode_body<64>(a);
}

unsigned grid_for(int64_t items) {
  const int64_t blocks = (items + 255) / 256;
  return (unsigned)(blocks < 16384 ? (blocks > 0 ? blocks : 1) : 16384);
}

}  // namespace

CacheSplit cache_split(const MimirCacheAttnParams& p) {
  CacheSplit s;
  const int G = p.num_kv_heads > 0 ? p.num_q_heads / p.num_kv_heads : 1;
  const int64_t R = (int64_t)p.seqlen * G;
  s.decode = R <= kDecRows;  // the decode kernels: 32-key wave tiles, one workgroup per CU
  s.n_rt = (int)((R + kRows - 1) / kRows);
  int max_kv = p.max_kv_len < p.cache_len ? p.max_kv_len : p.cache_len;
  if (max_kv < 1) max_kv = 1;
  const int tile_keys = s.decode ? kDecKeys : kKeys;
  const int tiles = (max_kv + tile_keys - 1) / tile_keys;
  s.groups = (int64_t)p.batch * p.num_kv_heads * s.n_rt;
  // workgroups to cover the chip: one per CU for the decode kernel, two for the other
  const int64_t target = (s.decode ? 1 : 2) * (int64_t)device_cu_count();
  int64_t splits = s.groups > 0 ? (target + s.groups - 1) / s.groups : 1;
  if (splits < 1) splits = 1;
  if (splits > tiles) splits = tiles;
  if (splits > kMaxSplits) splits = kMaxSplits;
  s.splits = (int)splits;
  s.units = s.groups * s.splits;
  // partial O, then (max, sum) per unit row, then the arrival counters
  s.workspace_bytes =
      s.splits > 1 ? (size_t)s.units * kRows * ((size_t)p.head_dim + 2) * sizeof(float) + (size_t)s.groups * 4 : 0;
  return s;
}

hipError_t launch_cache_attn_bf16(const MimirCacheAttnParams& p, hipStream_t stream) {
  const CacheSplit sp = cache_split(p);
  CacheArgs a;
  a.q = (const bf16_t*)p.q;
  a.kn = (const bf16_t*)p.k_new;
  a.vn = (const bf16_t*)p.v_new;
  a.ck = (bf16_t*)p.cache_k;
  a.cv = (bf16_t*)p.cache_v;
  a.out = (bf16_t*)p.out;
  a.cache_lengths = p.cache_lengths;
  a.batch_indices = p.batch_indices;
  a.q_sb = p.q_stride_batch; a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.kn_sb = p.kn_stride_batch; a.kn_st = p.kn_stride_token; a.kn_sh = p.kn_stride_head;
  a.vn_sb = p.vn_stride_batch; a.vn_st = p.vn_stride_token; a.vn_sh = p.vn_stride_head;
  a.ck_sb = p.ck_stride_batch; a.ck_st = p.ck_stride_token; a.ck_sh = p.ck_stride_head;
  a.cv_sb = p.cv_stride_batch; a.cv_st = p.cv_stride_token; a.cv_sh = p.cv_stride_head;
  a.o_sb = p.out_stride_batch; a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.B = p.batch;
  a.S = p.seqlen;
  a.L = p.cache_len;
  a.rows = p.cache_rows;
  a.Hkv = p.num_kv_heads;
  a.G = p.num_q_heads / p.num_kv_heads;
  a.causal = p.causal != 0;
  a.D = p.head_dim;
  a.idx64 = p.index_int64 != 0;
  a.n_rt = sp.n_rt;
  a.splits = sp.splits;
  a.scale_log2 = p.softmax_scale * kLog2e;
  a.part_o = (float*)p.workspace;
  a.part_ml = a.part_o + (size_t)sp.units * kRows * p.head_dim;
  a.counters = (int*)(a.part_ml + (size_t)sp.units * kRows * 2);
  a.n_counters = sp.splits > 1 ? (int)sp.groups : 0;
  if (sp.splits > 1 && p.workspace == nullptr) return hipErrorInvalidValue;
  const int64_t appends = (int64_t)a.B * a.S * a.Hkv * (a.D / 8);
  // units > 0 implies appends > 0, so the counters are always cleared before use
  if (appends > 0) hipLaunchKernelGGL(cache_append_kernel, dim3(grid_for(appends)), dim3(256), 0, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || sp.units == 0) return e;
  if (sp.decode) {
    if (p.head_dim == 128)
      hipLaunchKernelGGL(cache_decode_d128_kernel, dim3((unsigned)sp.units), dim3(kThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(cache_decode_d64_kernel, dim3((unsigned)sp.units), dim3(kThreads), 0, stream, a);
    return hipGetLastError();
  }
  if (p.head_dim == 128)
    hipLaunchKernelGGL(cache_attn_kernel<128>, dim3((unsigned)sp.units), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL(cache_attn_kernel<64>, dim3((unsigned)sp.units), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
