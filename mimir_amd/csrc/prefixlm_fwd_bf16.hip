// bf16 prefix-LM attention forward for gfx950 (MI355X).
//
// One workgroup = 4 waves = 128 query rows of one (sequence, query head); each
// wave owns 32 rows.  Workgroup r * Hq + h takes head h of entry r of the tile
// work list (prefixlm_prologue.hip): query tiles sorted by key range, longest first.
//
// The kernel computes S^T = K Q^T on v_mfma_f32_32x32x16_bf16 so that every lane
// holds one query column of the score tile: the softmax max/sum over keys is a
// per-lane reduction plus one v_permlane32_swap, the running max / sum / rescale
// factor are lane-local, and the probabilities P^T leave the accumulator already
// in the B-operand layout of O^T += V^T P^T.  V^T fragments come straight from
// the row-major V tile through ds_read_b64_tr_b16.  K/V tiles of 64 keys are
// staged in LDS (TileLayout: padded, row-permuted, bank-conflict-free) by direct
// buffer-to-LDS loads, double-buffered so that tile t + 1 streams in while tile
// t is consumed, with one barrier per tile.
//
// Tile classes follow the mask algebra j < kend(i) = max(p, i + 1): key tiles at
// or beyond a wave's largest kend are skipped, tiles entirely below its smallest
// kend run unmasked (the whole prefix block is dense), the rest are masked
// element-wise.  Reference semantics: flash_attention_prefixlm_dense.py:19-81;
// the Metal online-softmax forward flash_attention_prefixlm_mps.py:391-476 is the
// scalar ancestor of this loop (same m / l / lse = m + log(l) bookkeeping).
#include "prefixlm_common.h"

namespace {
using namespace mimir;

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBlockM = kWaves * 32;
constexpr int kBlockN = 64;

struct FwdArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  bf16_t* o;
  float* lse;
  const int32_t* prefix_lens;
  const int32_t* cu_seqlens;
  int64_t q_st, q_sh, k_st, k_sh, v_st, v_sh, o_st, o_sh, lse_sh;
  int T;             // packed length
  int Hq;
  int group;         // Hq / Hkv
  int total_seqlen;
  int is_causal;
  const int4* plan;  // (sequence, query tile, part | parts << 8 | span << 16, chunk slot), heaviest first (prefixlm_prologue.hip)
  int cap;           // entries of the list
  float scale;       // softmax scale
  float scale_log2;  // softmax scale * log2(e)
  const bf16_t* gate;  // optional sigmoid output gate [T, Hq, D]; y = round(round(sigmoid(gate)) * O)
  bf16_t* y;
  int64_t g_st, g_sh, y_st, y_sh;
  bf16_t* o_lo;        // optional low half: round(O - round(O)), O the fp32 output
  int64_t olo_st, olo_sh;
  const int* kscan;    // the prologue's K scan (split_mode AUTO)
  int split_mode;      // MimirSplitMode: P as bf16 hi + lo in O^T += V^T P^T
  int* split_flag;     // optional: the decision, for the backward
  int* chunk_ctr;      // arrival counter per (first chunk slot of a tile, q head)
  char* chunk_part;    // partials per (chunk slot, q head), chunk_slot_bytes(D) each
  RopeTab rope;        // optional RoPE of Q, applied to the loaded fragments
  bf16_t* q_rope;      // optional: the rotated Q rows, for the backward
  int64_t qr_st, qr_sh;
};

// Two LDS stages of one K tile and one V tile each.  Separate objects let the
// compiler see that reads of one stage never alias the loads into the other;
// declared apart from the tile loop's body so that both of a kernel's bodies
// (split and plain P) use the same LDS.  One set per kernel (kGated): objects
// that the called split body shares with one kernel only sit at fixed
// addresses, where objects shared by two kernels are found through a table.
template <int D>
struct FwdStages {
  bf16_t *k0, *v0, *k1, *v1;
};
template <int D, int kGated>
__device__ __forceinline__ FwdStages<D> fwd_stages() {
  using L = TileLayout<D>;
  __shared__ __attribute__((aligned(16))) bf16_t sK0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV0[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sK1[L::kElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV1[L::kElems];
  return FwdStages<D>{sK0, sV0, sK1, sV1};
}

// kSplit: P is not (0) / is (1) split.  The split changes the registers of the
// tile loop, so it is a compile-time choice; the kernel calls the split body as
// a function of its own (fwd_split_body).  (Both bodies inlined in one function,
// behind a uniform branch, made the plain one 10-17% slower.)
template <int D, int kGated, int kSplit>
__device__ __forceinline__ void fwd_body(const FwdArgs& a, uint64_t seg) {
  constexpr int DT = D / 32;  // 32-row d tiles of O^T
  constexpr int KS = D / 16;  // k-steps of S^T = K Q^T

  using L = TileLayout<D>;
  static_assert(kBlockN == 64, "one TileLayout tile per K / V block");
  const FwdStages<D> stages = fwd_stages<D, kGated>();
  bf16_t* const sK0 = stages.k0;
  bf16_t* const sV0 = stages.v0;
  bf16_t* const sK1 = stages.k1;
  bf16_t* const sV1 = stages.v1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hi = lane >> 5;

  // P as bf16 hi + lo in the P V product (the kernel picked this body by the
  // split decision): O, and the backward's delta = rowsum(dO * O), then carry no
  // rounding of P.  Workgroup 0 records the decision before anything can end it
  // early.
  if (a.split_flag != nullptr && blockIdx.x == 0 && tid == 0) *a.split_flag = kSplit;
  constexpr bool split = kSplit == 1;

  // Workgroup -> (list entry, head), see the grid in launch(): unit = entry *
  // Hkv + kv head on XCD unit % 8, its q heads at consecutive slots there.
  const int hkv = a.Hq / a.group;
  const int xcd = blockIdx.x % kXcds, slot = blockIdx.x / kXcds;
  const int unit = (slot / a.group) * kXcds + xcd;
  if (unit >= a.cap * hkv) return;
  const int rank = unit / hkv;
  const int h = (unit - rank * hkv) * a.group + slot % a.group;
  const int4 item = load_entry(a.plan, rank);
  if (item.x < 0) return;  // list padding
  const int s = item.x;
  const int mtile = item.y;
  const int part = item.z & 0xff, parts = (item.z >> 8) & 0xff, span = item.z >> 16;
  const SeqGeom g = load_seq<true>(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
  const int m0 = mtile * kBlockM;
  if (m0 >= g.nq) return;
  const int hk = h / a.group;

  const int wg_qend = min(m0 + kBlockM, g.nq);
  const int wg_kend = max(g.p, wg_qend);
  const int nkt_all = (wg_kend + kBlockN - 1) / kBlockN;
  // key tiles [kt0, nkt) of this part: the whole range unless the list cut it, then
  // the last parts `span` tiles each and the first the rest
  const int kt0 = part == 0 ? 0 : nkt_all - (parts - part) * span;
  const int nkt = nkt_all - (parts - 1 - part) * span;

  const int qa = m0 + wave * 32;
  const bool wave_active = qa < g.nq;
  const int w_kend_max = wave_active ? max(g.p, min(qa + 32, g.nq)) : 0;
  const int w_kend_min = max(g.p, qa + 1);
  const int qpos = qa + l32;
  const int kend_lane = kend_of(g.p, qpos);

  const __amdgpu_buffer_rsrc_t rq =
      make_rsrc(a.q + (int64_t)g.start * a.q_st + (int64_t)h * a.q_sh, rows_bytes(g.nq, a.q_st, D));
  const bf16_t* kseq = a.k + (int64_t)g.start * a.k_st + (int64_t)hk * a.k_sh;
  const bf16_t* vseq = a.v + (int64_t)g.start * a.v_st + (int64_t)hk * a.v_sh;
  const TileLoader<D, kWaves> ldk(a.k_st, wave, lane), ldv(a.v_st, wave, lane);

  // Tile copies walk the key tiles in order with running addresses (adds only).
  const bf16_t* i_k = kseq + (int64_t)kt0 * kBlockN * a.k_st;
  const bf16_t* i_v = vseq + (int64_t)kt0 * kBlockN * a.v_st;
  int i_rows = g.n - kt0 * kBlockN;
  auto issue_next = [&](bf16_t* tk, bf16_t* tv) {
    ldk.issue_at(i_k, rows_bytes32(i_rows, (uint32_t)a.k_st, D), tk);
    ldv.issue_at(i_v, rows_bytes32(i_rows, (uint32_t)a.v_st, D), tv);
    i_k += kBlockN * a.k_st;
    i_v += kBlockN * a.v_st;
    i_rows -= kBlockN;
  };
  if (kt0 < nkt) issue_next(sK0, sV0);

  // Q^T B-operand fragments: lane holds query qpos, d = 16*ks + 8*hi .. +7.
  bf16x8 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const uint32_t off = (uint32_t)(((int64_t)qpos * a.q_st + 16 * ks + 8 * hi) * 2);
    qf[ks] = __builtin_bit_cast(bf16x8, buf_load16(rq, off));
  }
  // RoPE: fragment ks (d = 16 ks + 8 hi ..) pairs with ks + KS / 2 (d + D / 2)
  // of the same lane.  Rows past the sequence read the last token's tables and
  // are never stored.
  if (a.rope.cos != nullptr) {
    const RopeTab rope = rope_at(seg, offsetof(FwdArgs, rope));
    const int64_t t = min(g.start + qpos, a.T - 1);
#pragma unroll
    for (int ks = 0; ks < KS / 2; ++ks) {
      bf16x4 y1[2], y2[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        f32x4 x1, x2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x1[e] = (float)qf[ks][4 * j + e];
          x2[e] = (float)qf[ks + KS / 2][4 * j + e];
        }
        rope_rotate4(rope, t, 16 * ks + 8 * hi + 4 * j, D / 2, x1, x2, y1[j], y2[j]);
      }
      qf[ks] = cat8(y1[0], y1[1]);
      qf[ks + KS / 2] = cat8(y2[0], y2[1]);
    }
  }
  // Gated store: round(sigmoid(gate)) of this lane's output elements, formed
  // before the tile loop so that neither the gate rows' latency nor the
  // sigmoid lands in the epilogue (rows >= nq read as 0 and are not stored).
  bf16x4 sgate[kGated ? DT * 4 : 1];
  if constexpr (kGated != 0) {
    const __amdgpu_buffer_rsrc_t rgate =
        make_rsrc(a.gate + (int64_t)g.start * a.g_st + (int64_t)h * a.g_sh, rows_bytes(g.nq, a.g_st, D));
#pragma unroll
    for (int i = 0; i < DT * 4; ++i) {
      const int col = 32 * (i >> 2) + 8 * (i & 3) + 4 * hi;
      const uint32_t off = (uint32_t)(((int64_t)qpos * a.g_st + col) * 2);
      const bf16x4 gv = __builtin_bit_cast(bf16x4, __builtin_amdgcn_raw_buffer_load_b64(rgate, off, 0, 0));
      f32x4 sv;
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = sigmoid_bf16((float)gv[e]);
      sgate[i] = __builtin_convertvector(sv, bf16x4);
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c2 = a.scale_log2;

  const TileLanes<D> tl(lane);

  // One 64-key tile; `masked` selects the element-wise mask (tiles that reach
  // past some row's kend).  A compile-time split into masked / unmasked bodies
  // was measured: the extra code copies push head_dim 128 over 256 VGPRs.
  auto compute = [&](bool masked, int kt, const bf16_t* sK, const bf16_t* sV) {
    const int kb = kt * kBlockN;

    // S^T = K Q^T for 64 keys: two 32-key sub-tiles.
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

    if (masked) {
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
    // Lazy rescaling: the reference max only moves when the running max grows by
    // more than 2^8 in probability terms (always on the first tile, where m_run is
    // -inf).  In between, probabilities stay below 256, exact in fp32 and in bf16's
    // range; the final 1/l uses the same reference, so the result is unchanged.
    // A part of a cut key range can meet a row's masked keys before any visible
    // one: the row keeps m_run = -inf (alpha 1, probabilities exp2(-inf) = 0).
    const float m_cand = fmaxf(m_run, mx);
    const bool grow = (m_cand - m_run) * c2 > 8.f;
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
      const float alpha = grow ? fast_exp2((m_run - m_cand) * c2) : 1.f;
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
      if (grow) m_run = m_cand;
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

    // P^T B-operand fragments (16 keys each), key order matching the V^T reads;
    // split: the low halves too, one more MFMA per V^T fragment.
    bf16x8 pf[4], pl[split ? 4 : 1];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int mt = kk >> 1, s8 = (kk & 1) * 8;
      f32x8 t;
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = st[mt][s8 + e];
      pf[kk] = to_bf16x8(t);
      if constexpr (split) pl[kk] = lo_half(t, pf[kk]);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16_t* vp = &sV[tl.tr_base + kk * 16 * L::kRowElems + dt * 32];
        const bf16x4 v0 = lds_read_tr16(vp);
        const bf16x4 v1 = lds_read_tr16(vp + L::kTrSecond);
        const bf16x8 vt = cat8(v0, v1);
        oacc[dt] = mfma32(vt, pf[kk], oacc[dt]);
        if constexpr (split) oacc[dt] = mfma32(vt, pl[kk], oacc[dt]);
      }
    }
  };

  auto step = [&](int kt, const bf16_t* sK, const bf16_t* sV) {
    const int kb = kt * kBlockN;
    if (!wave_active || kb >= w_kend_max) return;
    compute(kb + kBlockN > w_kend_min, kt, sK, sV);
  };

  for (int kt = kt0; kt < nkt; kt += 2) {
    wait_vmem();
    __syncthreads();
    if (kt + 1 < nkt) issue_next(sK1, sV1);
    step(kt, sK0, sV0);
    if (kt + 1 >= nkt) break;
    wait_vmem();
    __syncthreads();
    if (kt + 2 < nkt) issue_next(sK0, sV0);
    step(kt + 1, sK1, sV1);
  }

  // A part of a cut key range: publish the partial (unnormalized O, running max
  // and sum per lane) in its chunk slot; the last part of the tile to arrive
  // merges all of them, in part order, and runs the epilogue.
  if (__builtin_expect(parts > 1, 0)) {
    __shared__ int later;
    constexpr int kDevScope = 16;  // buffer cache policy: coherent at device scope
    constexpr uint32_t kOBytes = (uint32_t)D * 128 * 4;
    const int slot0 = item.w - part;
    const size_t slot_bytes = chunk_slot_bytes(D);
    char* const mine = a.chunk_part + ((size_t)item.w * a.Hq + h) * slot_bytes;
    {
      const __amdgpu_buffer_rsrc_t r = make_rsrc(mine, (uint32_t)slot_bytes);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 v = {oacc[dt][4 * rg], oacc[dt][4 * rg + 1], oacc[dt][4 * rg + 2], oacc[dt][4 * rg + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, v), r,
                                                 (uint32_t)((((wave * DT + dt) * 4 + rg) * 64 + lane) * 16), 0,
                                                 kDevScope);
        }
      const f32x2 ml = {m_run, l_run};
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(i32x2, ml), r,
                                            kOBytes + (uint32_t)((wave * 64 + lane) * 8), 0, kDevScope);
    }
    __asm__ volatile("" ::: "memory");
    wait_vmem();  // the slot stores are complete
    __syncthreads();
    if (tid == 0) {
      int* const ctr = a.chunk_ctr + (size_t)slot0 * a.Hq + h;
      const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (prev == parts - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      later = prev == parts - 1;
    }
    __syncthreads();
    if (!later) return;
    // Merge: max of the parts' reference maxima, then the sum of their sums and
    // O accumulators rescaled to it (a part with no key for the row has max -inf).
    auto slot_of = [&](int q) {
      return make_rsrc(a.chunk_part + ((size_t)(slot0 + q) * a.Hq + h) * slot_bytes, (uint32_t)slot_bytes);
    };
    float m_all = -INFINITY;
    for (int q = 0; q < parts; ++q) {
      const i32x2 v = __builtin_amdgcn_raw_buffer_load_b64(slot_of(q), kOBytes + (uint32_t)((wave * 64 + lane) * 8),
                                                           0, kDevScope);
      m_all = fmaxf(m_all, __builtin_bit_cast(f32x2, v)[0]);
    }
    float l_all = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
    for (int q = 0; q < parts; ++q) {
      const __amdgpu_buffer_rsrc_t r = slot_of(q);
      const f32x2 ml = __builtin_bit_cast(
          f32x2, __builtin_amdgcn_raw_buffer_load_b64(r, kOBytes + (uint32_t)((wave * 64 + lane) * 8), 0, kDevScope));
      const float f = ml[0] == -INFINITY ? 0.f : fast_exp2((ml[0] - m_all) * c2);
      l_all += ml[1] * f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          const f32x4 v = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         r, (uint32_t)((((wave * DT + dt) * 4 + rg) * 64 + lane) * 16), 0, kDevScope));
#pragma unroll
          for (int e = 0; e < 4; ++e) oacc[dt][4 * rg + e] += v[e] * f;
        }
    }
    m_run = m_all;
    l_run = l_all;
  }

  // Epilogue: each wave stages its 32 output rows (and the gated rows) in LDS --
  // one K / V stage object per wave, free once every wave is past the tile
  // loop -- and stores whole rows, kRowsPerInst rows of D * 2 contiguous bytes
  // per store instruction instead of 32 pieces of 16 bytes.
  __syncthreads();
  if (!wave_active) return;
  const float l_tot = xor32_sum(l_run);
  const float inv = 1.f / l_tot;
  constexpr int kPitch = D + 8;                 // elements; rows stay 16-byte aligned
  constexpr int kUnits = D / 8;                 // 16-byte units per row
  constexpr int kRowsPerInst = 64 / kUnits;
  static_assert((kGated ? 2 : 1) * 32 * kPitch <= L::kElems, "a wave's rows fit its stage object");
  bf16_t* const stage = wave == 0 ? sK0 : wave == 1 ? sV0 : wave == 2 ? sK1 : sV1;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 t;
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = oacc[dt][4 * rg + e] * inv;
      *(bf16x4*)&stage[l32 * kPitch + 32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(t, bf16x4);
      if constexpr (kGated != 0) {
        // Sigmoid output gate in the store (layers.py:239): y = round(s * O) with
        // s = round(sigmoid(gate)) and O the rounded attention output, as the
        // reference's bf16 torch.sigmoid(gate) * attn_output rounds them.
        f32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = (float)sgate[4 * dt + rg][e] * round_to(t[e], bf16_t());
        *(bf16x4*)&stage[(32 + l32) * kPitch + 32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(y, bf16x4);
      }
    }
  if (hi == 0 && a.lse != nullptr && qpos < g.nq)
    a.lse[(int64_t)h * a.lse_sh + g.start + qpos] = m_run * a.scale + fast_log2(l_tot) * kLn2;
  // The LDS unit runs one wave's accesses in order: the reads below see the writes above.
  __asm__ volatile("" ::: "memory");
  const int u = lane % kUnits;
  bf16_t* const obase = a.o + (int64_t)(g.start + qa) * a.o_st + (int64_t)h * a.o_sh + u * 8;
  bf16_t* ybase = nullptr;
  if constexpr (kGated != 0) ybase = a.y + (int64_t)(g.start + qa) * a.y_st + (int64_t)h * a.y_sh + u * 8;
#pragma unroll
  for (int j = 0; j < 32 / kRowsPerInst; ++j) {
    const int r = j * kRowsPerInst + lane / kUnits;
    const bf16x8 ov = *(const bf16x8*)&stage[r * kPitch + u * 8];
    bf16x8 yv;
    if constexpr (kGated != 0) yv = *(const bf16x8*)&stage[(32 + r) * kPitch + u * 8];
    if (qa + r < g.nq) {
      *(bf16x8*)&obase[(int64_t)r * a.o_st] = ov;
      if constexpr (kGated != 0) *(bf16x8*)&ybase[(int64_t)r * a.y_st] = yv;
    }
  }
  // The rotated Q rows (RoPE in the kernel) for the backward: another round
  // through the staging rows, whole rows per store as for O.
  bf16_t* const q_rope = kernarg_at<bf16_t*>(seg, offsetof(FwdArgs, q_rope));
  if (q_rope != nullptr) {
    const int64_t qr_st = kernarg_at<int64_t>(seg, offsetof(FwdArgs, qr_st));
    const int64_t qr_sh = kernarg_at<int64_t>(seg, offsetof(FwdArgs, qr_sh));
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) *(bf16x8*)&stage[l32 * kPitch + 16 * ks + 8 * hi] = qf[ks];
    __asm__ volatile("" ::: "memory");
    bf16_t* const rbase = q_rope + (int64_t)(g.start + qa) * qr_st + (int64_t)h * qr_sh + u * 8;
#pragma unroll
    for (int j = 0; j < 32 / kRowsPerInst; ++j) {
      const int r = j * kRowsPerInst + lane / kUnits;
      const bf16x8 v = *(const bf16x8*)&stage[r * kPitch + u * 8];
      if (qa + r < g.nq) *(bf16x8*)&rbase[(int64_t)r * qr_st] = v;
    }
  }
  // The low halves: with a recorded decision only when split (the backward
  // reads them only then), otherwise always.
  if (a.o_lo == nullptr || (a.split_flag != nullptr && !split)) return;
  // Low halves, a second round through the same staging rows (the reads above
  // are complete before these writes reach LDS: one wave's LDS accesses run in order).
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int rg = 0; rg < 4; ++rg) {
      f32x4 lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float t = oacc[dt][4 * rg + e] * inv;
        lo[e] = t - round_to(t, bf16_t());
      }
      *(bf16x4*)&stage[l32 * kPitch + 32 * dt + 8 * rg + 4 * hi] = __builtin_convertvector(lo, bf16x4);
    }
  __asm__ volatile("" ::: "memory");
  bf16_t* const lbase = a.o_lo + (int64_t)(g.start + qa) * a.olo_st + (int64_t)h * a.olo_sh + u * 8;
#pragma unroll
  for (int j = 0; j < 32 / kRowsPerInst; ++j) {
    const int r = j * kRowsPerInst + lane / kUnits;
    const bf16x8 lv = *(const bf16x8*)&stage[r * kPitch + u * 8];
    if (qa + r < g.nq) *(bf16x8*)&lbase[(int64_t)r * a.olo_st] = lv;
  }
}

// The split body (P as bf16 hi + lo) in a function of its own, which the kernel
// calls when the split is on: the plain body, inlined in the kernel, keeps the
// registers and code of a kernel of its own.  It reads its arguments from the
// kernel's argument segment `seg` (a reference to the kernel's by-value
// argument would make the compiler copy it to the stack for both bodies).
template <int D, int kGated>
__device__ __attribute__((noinline)) void fwd_split_body(uint64_t seg) {
  seg = uniform_segment(seg);
  fwd_body<D, kGated, 1>(segment_args<FwdArgs>(seg), seg);
}
// One launch for every split mode: the decision (the K scan's with AUTO) picks
// the body.  Plain and gated stores are separate kernels, so that the gate's
// pointers stay out of the plain kernel's scalar registers.
template <int D, int kGated>
__device__ __forceinline__ void fwd_kernel_body(const FwdArgs& a) {
  if (split_decision(a.split_mode, a.kscan, nullptr, threadIdx.x & 63))
    fwd_split_body<D, kGated>(kernel_segment());
  else
    fwd_body<D, kGated, 0>(a, kernel_segment());
}
// Waves per SIMD (= workgroups per CU) the kernel runs at: head_dim 64 four
// (gated: three), head_dim 128 two.  Pinned as both the least and the most: the
// register budget must allow that many, and the called split body, whose
// occupancy the compiler cannot bound by the kernel's LDS, is scheduled for
// the same count (with only the least given it aimed at more waves and
// serialized its LDS operand reads to save registers).
template <int D, int kGated>
constexpr int kFwdWaves = D == 64 ? (kGated ? 3 : 4) : 2;
template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(kFwdWaves<D, 0>, kFwdWaves<D, 0>))) void fwd_bf16_kernel(const FwdArgs a) {
  fwd_kernel_body<D, 0>(a);
}
template <int D>
__global__ __attribute__((amdgpu_flat_work_group_size(kThreads, kThreads),
                          amdgpu_waves_per_eu(kFwdWaves<D, 1>, kFwdWaves<D, 1>))) void fwd_bf16_gated_kernel(const FwdArgs a) {
  fwd_kernel_body<D, 1>(a);
}

template <int D>
hipError_t launch(const MimirPrefixLMFwdParams& p, Prologue pro, hipStream_t stream) {
  FwdArgs a;
  a.q = (const bf16_t*)p.q;
  a.k = (const bf16_t*)p.k;
  a.v = (const bf16_t*)p.v;
  a.o = (bf16_t*)p.out;
  a.lse = p.lse;
  a.prefix_lens = p.prefix_lens;
  a.cu_seqlens = p.cu_seqlens;
  a.q_st = p.q_stride_token; a.q_sh = p.q_stride_head;
  a.k_st = p.k_stride_token; a.k_sh = p.k_stride_head;
  a.v_st = p.v_stride_token; a.v_sh = p.v_stride_head;
  a.o_st = p.out_stride_token; a.o_sh = p.out_stride_head;
  a.lse_sh = p.lse_stride_head;
  a.T = p.total_tokens;
  a.Hq = p.num_q_heads;
  a.group = p.num_q_heads / p.num_kv_heads;
  a.total_seqlen = p.total_seqlen;
  a.is_causal = p.is_causal;
  a.scale = p.softmax_scale;
  a.scale_log2 = p.softmax_scale * kLog2e;
  a.gate = (const bf16_t*)p.gate;
  a.y = (bf16_t*)p.gated_out;
  a.g_st = p.gate_stride_token; a.g_sh = p.gate_stride_head;
  a.y_st = p.gated_out_stride_token; a.y_sh = p.gated_out_stride_head;
  a.o_lo = (bf16_t*)p.out_lo;
  a.olo_st = p.out_lo_stride_token; a.olo_sh = p.out_lo_stride_head;
  a.split_mode = p.split_mode;
  a.split_flag = p.split_flag;
  a.rope = RopeTab{p.rope_cos, p.rope_sin, p.rope_stride_token};
  a.q_rope = (bf16_t*)p.q_rope;
  a.qr_st = p.q_rope_stride_token; a.qr_sh = p.q_rope_stride_head;
  static_assert(kBlockM == kPlanTile, "work-list tiles are the forward's query tiles");
  const int cap_items = plan_capacity(p.total_tokens, p.numseqs, p.max_seqlen_all);
  // key-range parts when the workspace has room for their slots (small grids)
  const FwdWorkspace full = fwd_workspace_layout(cap_items, p.num_q_heads, D, true);
  const bool chunks = full.chunk_slots > 0 && p.workspace_bytes >= full.total;
  const FwdWorkspace ws = chunks ? full : fwd_workspace_layout(cap_items, p.num_q_heads, D, false);
  const int cap = ws.list_cap;
  int4* plan = (int4*)((char*)p.workspace + ws.list);
  a.plan = plan;
  a.cap = cap;
  a.kscan = (const int*)((char*)p.workspace + ws.kscan);
  a.chunk_ctr = chunks ? (int*)((char*)p.workspace + ws.ctr) : nullptr;
  a.chunk_part = chunks ? (char*)p.workspace + ws.part : nullptr;
  if (cap > 0) {
    pro.plan[pro.nplan] = plan_args(p.cu_seqlens, p.prefix_lens, p.numseqs, p.total_seqlen, p.is_causal,
                                    p.total_tokens, /*kind=*/2, a.group, cap, plan);
    if (chunks) {
      pro.plan[pro.nplan].split_heads = p.num_q_heads;
      pro.plan[pro.nplan].slots = kChunkWgs;
      // parts of 1.25 x the per-slot average: XXS forward 5.5% faster than at 1.0
      // (1.5: 4%); the dQ list keeps 1.0, where larger parts measured slower
      pro.plan[pro.nplan].span_pct = 125;
      pro.plan[pro.nplan].max_pairs = ws.chunk_slots;
      pro.plan[pro.nplan].zero = a.chunk_ctr;
      pro.plan[pro.nplan].n_zero = ws.chunk_slots * p.num_q_heads;
    }
    ++pro.nplan;
    if (p.split_mode == MIMIR_SPLIT_AUTO) {  // the K scan behind the split decision
      pro.kscan = kscan_args(a.k, a.k_st, a.k_sh, a.T, p.num_kv_heads, D, p.softmax_scale, (int*)a.kscan,
                             p.cu_seqlens, p.numseqs);
      pro.has_kscan = 1;
    }
  }
  hipError_t e = launch_prologue(pro, stream);
  if (e != hipSuccess || cap == 0) return e;
  // Workgroup b runs on XCD b % 8 (the dispatcher deals workgroups to the XCDs
  // round-robin).  Unit u = list entry * Hkv + kv head goes to XCD u % 8 and its
  // `group` q heads to consecutive slots there: the heads that read the same K /
  // V tiles stream them through one XCD's L2 at about the same time, and each
  // XCD keeps to a few kv heads.  On the packed 8 x 2048 GQA batch (Hq 16, Hkv 4)
  // this cuts the kernel's HBM reads from 2.9x to 1.1x the compulsory Q, K, V
  // bytes (the time does not change: the kernel is not HBM-bound).  Slots past
  // the last unit exit at once.
  const int64_t units = (int64_t)cap * p.num_kv_heads;
  const dim3 grid((unsigned)(((units + kXcds - 1) / kXcds) * kXcds * a.group));
  hipLaunchKernelGGL(a.gate != nullptr ? fwd_bf16_gated_kernel<D> : fwd_bf16_kernel<D>, grid, dim3(kThreads), 0,
                     stream, a);
  return hipGetLastError();
}

}  // namespace

bool mimir_bf16_head_dim_supported(int d) { return d == 64 || d == 128; }

hipError_t mimir_launch_fwd_bf16(const MimirPrefixLMFwdParams& p, Prologue pro, hipStream_t stream) {
  switch (p.head_dim) {
    case 64: return launch<64>(p, pro, stream);
    case 128: return launch<128>(p, pro, stream);
    default: return hipErrorInvalidValue;
  }
}
