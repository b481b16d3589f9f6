// The small per-call work in front of the tile loops, in one launch: the tile
// work lists, the backward's delta / lse * log2(e) rows and the padding-row
// fills.  Separate launches cost a few microseconds each of mostly idle GPU;
// here the workgroups of the three jobs share one grid and run side by side.
//
//   workgroups [0, nplan)               one tile work list each
//   then [0, kscan_blocks)               K magnitude scan (the split decision)
//   then [0, delta_blocks)               delta = rowsum(O * dO), lse * log2(e)
//   then nfill x [0, fill_blocks)        zero rows outside every sequence
// (the single-workgroup lists and the scan go first: they are latency-bound,
// and dispatched behind thousands of delta workgroups they would end last)
//
// Tile work lists: which (sequence, 128-row tile) each workgroup of the forward,
// dQ and dK/dV kernels takes, heaviest first.  Dispatching (column, tile row)
// rectangles row by row only approximates heaviest-first: on batches of a few
// 2k sequences the last workgroups to start were still large and the kernels
// ended on long tails.  One workgroup computes every item's cost from the
// metadata on the device (no host copy of cu_seqlens / prefix_lens),
// counting-sorts the items by cost, descending, into the caller's workspace and
// pads the list with (-1, -1).  Workgroup r * H + h of the consumer takes list
// entry r for head h: the H heads of one item run back to back and the dispatch
// order is longest-processing-time first.  The order inside one cost bucket
// follows LDS atomics and may differ from call to call; every item writes its
// own outputs, so results do not.
//
// Costs, in 64-row tiles of the inner loop:
//   query tiles (forward, dQ):  key tiles up to kend of the tile's last row,
//                               ceil(max(p, min(m0 + 128, nq)) / 64)
//   key tiles (dK / dV):        G * query tiles from qstart(first key),
//                               G * ceil((nq - qstart(kb0)) / 64), 0 if none
//
// Padding rows: rows that belong to no sequence, or lie at/after total_seqlen,
// are outputs of the operator too: O = 0, lse = -inf, dQ = 0
// (flash_attention_prefixlm_dense.py:43,79-80).  dK/dV rows outside every
// sequence are 0; key rows inside a sequence are written by the dK/dV kernel
// even at/after total_seqlen, since they remain keys there.  The fills touch
// only rows the tile kernels never write, so they may run before them.
#include "prefixlm_common.h"

namespace mimir {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kPlanBuckets = 4096;  // costs above kPlanBuckets - 1 share the last bucket
constexpr int kBucketsPerThread = kPlanBuckets / kThreads;
constexpr int kFillRows = 16;
constexpr int kFillWgs = 128;  // fill workgroups per target, at most

struct PrologueArgs {
  PlanArgs plan[2];
  DeltaArgs delta;
  KScanArgs kscan;
  FillArgs fill[3];
  int nplan, delta_blocks, kscan_blocks, nfill, fill_blocks;
};

// Exclusive prefix sum of v over the workgroup; `total` receives the sum.
__device__ int block_exclusive_scan(int v, int* wave_sums, int& total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) wave_sums[w] = x;
  __syncthreads();
  int before = 0;
  total = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const int s = wave_sums[i];
    before += i < w ? s : 0;
    total += s;
  }
  __syncthreads();  // wave_sums is reused by the next scan
  return before + x - v;
}

// Cost of tile t in 64-row steps of the consumer's loop (for kind 1 exactly
// its iteration count G * query tiles).
__device__ __forceinline__ int item_cost(int p, int nq, int kind, int group, int t) {
  if (kind != 1) {
    const int kend = max(p, min(t * kPlanTile + kPlanTile, nq));
    return (kend + 63) / 64;
  }
  const int q0 = qstart_of(p, t * kPlanTile);
  return nq > q0 ? group * ((nq - q0 + 63) / 64) : 0;
}

__device__ __forceinline__ int bucket_of(int cost) { return min(cost, kPlanBuckets - 1); }
// LDS slot of bucket b: one padding word every 16 buckets, so that the 16
// consecutive buckets each thread owns in bucket_starts sit in distinct banks
// across the wave.
constexpr int kHistSlots = kPlanBuckets + kPlanBuckets / 16;
__device__ __forceinline__ int bucket_slot(int b) { return b + (b >> 4); }
__device__ __forceinline__ int hist_slot(int cost) { return bucket_slot(bucket_of(cost)); }

struct PlanSmem {
  int hist[kHistSlots];
  int first_item[kThreads];  // per sequence of the current chunk
  int p[kThreads], nq[kThreads];
  int wave_sums[kWaves];
  double wave_dsums[kWaves];
  int cut, pairs;
  int chunk_items;  // items of the last chunk of sequences walked
};

__device__ __forceinline__ void put_item(const PlanArgs& a, int pos, int s, int t, int part, int pair) {
  if (pos >= a.cap) return;
  if (a.kind == 0)
    ((int2*)a.items)[pos] = make_int2(s, t);
  else
    ((int4*)a.items)[pos] = make_int4(s, t, part, pair);
}

// n consecutive indices from *counter for each lane of the wave (0 for none):
// a wave-wide exclusive scan and one atomic per wave.  Every lane of the wave
// must call it.
__device__ __forceinline__ int wave_alloc(int* counter, int n) {
  const int lane = threadIdx.x & 63;
  int x = n;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  int base = 0;
  if (lane == 63 && x > 0) base = atomicAdd(counter, x);
  base = __shfl(base, 63, 64);
  return base + x - n;
}

// Parts of a kind-2 item of cost c cut at `span` key tiles per part (0: no
// chunking): the last parts run `span` tiles each, the first the rest, so that
// the cut leaves whole-slot parts and one remainder for the end of the list.
__device__ __forceinline__ int chunk_parts(int c, int span) {
  if (span <= 0 || c <= span) return 1;
  const int n = (c + span - 1) / span;
  return n < kChunkMax ? n : kChunkMax;
}

// Visits every (sequence, tile) item, 256 sequences at a time: a scan of the
// tile counts gives each sequence its first item, then the items are dealt to
// the threads one each, so a single long sequence is spread over the workgroup
// too.  Items costing `cut` or more count as two halves.  Without kScatter the
// visit adds each item (or half) to its cost bucket; with kScatter it takes the
// next position of that bucket and writes the entry.  Kind 2 with `span` > 0
// cuts items into chunk_parts(cost, span) parts instead.  With `reuse` (only
// for numseqs <= kThreads, after a walk of the same list) the sequences' first
// items and geometry are still in `sm` and are not loaded again; `pre` is this
// thread's sequence of the first chunk, loaded by the caller ahead of time.
// Returns this thread's share of the total cost.
template <bool kScatter>
__device__ double walk_items(const PlanArgs& a, PlanSmem& sm, int cut, int span = 0, bool reuse = false,
                             const SeqGeom* pre = nullptr, int* items = nullptr) {
  double cost_sum = 0.0;
  if (items != nullptr) *items = 0;
  for (int base = 0; base < a.numseqs; base += kThreads) {
    int total;
    if (reuse) {
      total = sm.chunk_items;
    } else {
      const int s = base + (int)threadIdx.x;
      int nt = 0, p = 0, nq = 0;
      if (s < a.numseqs) {
        const SeqGeom g = base == 0 && pre != nullptr
                              ? *pre
                              : load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
        nt = ((a.kind != 1 ? g.nq : g.n) + kPlanTile - 1) / kPlanTile;
        p = g.p;
        nq = g.nq;
      }
      const int first = block_exclusive_scan(nt, sm.wave_sums, total);
      sm.first_item[threadIdx.x] = first;
      sm.p[threadIdx.x] = p;
      sm.nq[threadIdx.x] = nq;
      if (threadIdx.x == 0) sm.chunk_items = total;
      __syncthreads();
    }
    if (items != nullptr) *items += total;
    // Uniform trip count (every lane runs every round), so that the chunk slots
    // and pair indices are dealt by one atomic per wave instead of one per item.
    for (int i0 = 0; i0 < total; i0 += kThreads) {
      const int i = i0 + (int)threadIdx.x;
      const bool valid = i < total;
      // the last sequence of the chunk whose first item is <= i owns item i
      int j = 0, t = 0, c = 0;
      if (valid) {
#pragma unroll
        for (int step = kThreads / 2; step > 0; step >>= 1)
          if (sm.first_item[j + step] <= i) j += step;
        t = i - sm.first_item[j];
        c = item_cost(sm.p[j], sm.nq[j], a.kind, a.group, t);
        cost_sum += (double)c;
      }
      const int parts = valid && a.kind == 2 ? chunk_parts(c, span) : 1;
      int slot = 0;  // first chunk slot (kind 2 parts) or pair index (kind 1 halves)
      int spos = 0;  // kind 2: position (scatter) of the item's span-tile parts 1 ..
      if (a.kind == 2 && span > 0) {  // uniform
        const int n = valid && parts > 1 ? parts : 0;
        if (kScatter) slot = wave_alloc(&sm.pairs, n);
        // the span-tile parts of every cut item share one bucket: one LDS atomic
        // per wave (per-lane atomics on one word serialize)
        spos = wave_alloc(&sm.hist[hist_slot(span)], n > 0 ? n - 1 : 0);
      } else if (kScatter && a.kind != 2 && cut != 0x7fffffff) {  // uniform
        slot = wave_alloc(&sm.pairs, valid && a.kind == 1 && c >= cut ? 1 : 0);
      }
      if (!valid) continue;
      if (parts > 1) {
        const int c0 = c - (parts - 1) * span;  // the first part's tiles, the others `span`
        const int z = (parts << 8) | (span << 16);
        if constexpr (kScatter) {  // parts 1.. take consecutive positions; every part its slot
          put_item(a, atomicAdd(&sm.hist[hist_slot(c0)], 1), base + j, t, z, slot);
          for (int q = 1; q < parts; ++q) put_item(a, spos + q - 1, base + j, t, q | z, slot + q);
        } else {
          atomicAdd(&sm.hist[hist_slot(c0)], 1);
        }
      } else if (a.kind == 2) {
        if constexpr (kScatter) {
          put_item(a, atomicAdd(&sm.hist[hist_slot(c)], 1), base + j, t, 1 << 8, -1);
        } else {
          atomicAdd(&sm.hist[hist_slot(c)], 1);
        }
      } else if (c >= cut) {
        const int c1 = span > 0 ? span : c / 2, c2 = c - c1;
        if constexpr (kScatter) {  // half | first step of half 2 << 8 (0: the middle)
          put_item(a, atomicAdd(&sm.hist[hist_slot(c1)], 1), base + j, t, 1 | (span << 8), slot);
          put_item(a, atomicAdd(&sm.hist[hist_slot(c2)], 1), base + j, t, 2 | (span << 8), slot);
        } else {
          atomicAdd(&sm.hist[hist_slot(c1)], 1);
          atomicAdd(&sm.hist[hist_slot(c2)], 1);
        }
      } else if constexpr (kScatter) {
        put_item(a, atomicAdd(&sm.hist[hist_slot(c)], 1), base + j, t, 0, -1);
      } else {
        atomicAdd(&sm.hist[hist_slot(c)], 1);
      }
    }
    __syncthreads();  // the chunk arrays are rewritten by the next chunk
  }
  return cost_sum;
}

// Turns the bucket counts into start positions in descending cost order
// (bucket c starts after all items of cost > c) and returns the item count.
// Thread i owns buckets kPlanBuckets-1-16i down to kPlanBuckets-16-16i.  With
// `max_pairs` > 0 it also finds the split cut: the smallest bucket above
// `threshold` whose items and all heavier ones number at most max_pairs.
__device__ int bucket_starts(PlanSmem& sm, double threshold, int max_pairs) {
  int cnt[kBucketsPerThread];
  int local = 0;
#pragma unroll
  for (int j = 0; j < kBucketsPerThread; ++j) {
    cnt[j] = sm.hist[bucket_slot(kPlanBuckets - 1 - (kBucketsPerThread * threadIdx.x + j))];
    local += cnt[j];
  }
  int total;
  int run = block_exclusive_scan(local, sm.wave_sums, total);
  int cut = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < kBucketsPerThread; ++j) {
    const int b = kPlanBuckets - 1 - (kBucketsPerThread * threadIdx.x + j);
    sm.hist[bucket_slot(b)] = run;  // becomes the next free position of bucket b
    run += cnt[j];     // items of cost >= b
    if (max_pairs > 0 && (double)b > threshold && run <= max_pairs) cut = b;
  }
  if (max_pairs > 0) {  // uniform
    // the wave's minimum first, then one LDS atomic per wave: every thread's
    // atomic on the one word serialized to ~2.5 us
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cut = min(cut, __shfl_xor(cut, off, 64));
    if ((threadIdx.x & 63) == 0 && cut != 0x7fffffff) atomicMin(&sm.cut, cut);
  }
  __syncthreads();
  return total;
}

__device__ double block_sum(double v, PlanSmem& sm) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  if ((threadIdx.x & 63) == 0) sm.wave_dsums[threadIdx.x >> 6] = v;
  __syncthreads();
  double total = 0.0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) total += sm.wave_dsums[i];
  return total;
}

// A query-tile list (kind 2: the forward's, dQ's): counted once (items and
// cost); if the grid is small (fewer workgroups than a.slots resident at once)
// the items costing more than the per-workgroup average of one round (the
// span, in whole key tiles) are cut into parts (chunk_parts) and the counts are
// redone with the parts; then the bucket positions are scanned and the list is
// written.  A cut item of cost c > span has ceil(c / span) < 2 c / span parts,
// so the parts of all items number fewer than 2 * a.slots / a.split_heads <=
// a.max_pairs: the chunk slots suffice.
// The first chunk's sequence geometry, loaded before the zeroing so that its
// latency overlaps it.
__device__ __forceinline__ SeqGeom prefetch_seq(const PlanArgs& a) {
  SeqGeom g{};
  if ((int)threadIdx.x < a.numseqs)
    g = load_seq(a.cu_seqlens, a.prefix_lens, threadIdx.x, a.total_seqlen, a.is_causal, a.T);
  return g;
}

__device__ void plan_block_chunks(const PlanArgs& a, PlanSmem& sm) {
  const SeqGeom pre = prefetch_seq(a);
  for (int i = threadIdx.x; i < kHistSlots; i += kThreads) sm.hist[i] = 0;
  if (threadIdx.x == 0) sm.pairs = 0;
  for (int i = threadIdx.x; i < a.n_zero; i += kThreads) a.zero[i] = 0;
  __syncthreads();
  int items = 0;
  const double mine = walk_items<false>(a, sm, 0x7fffffff, 0.0, false, &pre, &items);
  const bool reuse = a.numseqs <= kThreads;  // one chunk of sequences: still in sm
  int total;
  int span = 0;
  if (a.max_pairs > 0 && a.split_heads > 0 && (int64_t)items * a.split_heads < (int64_t)a.slots) {
    // small grid: recount with the cut items' parts (the first counts are not used)
    const double target = block_sum(mine, sm) * a.split_heads / a.slots * (a.span_pct < 100 ? 100 : a.span_pct) / 100.0;
    span = target > (double)kChunkMinCost ? (int)ceil(target) : kChunkMinCost;
    for (int i = threadIdx.x; i < kHistSlots; i += kThreads) sm.hist[i] = 0;
    __syncthreads();
    walk_items<false>(a, sm, 0x7fffffff, span, reuse);
  }
  total = bucket_starts(sm, 0.0, 0);
  walk_items<true>(a, sm, 0x7fffffff, span, reuse);
  for (int i = total + threadIdx.x; i < a.cap; i += kThreads) put_item(a, i, -1, -1, 0, -1);
}

__device__ void plan_block(const PlanArgs& a) {
  __shared__ PlanSmem sm;
  if (a.kind == 2) {
    plan_block_chunks(a, sm);
    return;
  }
  const bool split = a.kind == 1 && a.split_heads > 0 && a.max_pairs > 0 && a.slots > 0;
  const SeqGeom pre = prefetch_seq(a);
  for (int i = threadIdx.x; i < kHistSlots; i += kThreads) sm.hist[i] = 0;
  if (threadIdx.x == 0) {
    sm.cut = 0x7fffffff;
    sm.pairs = 0;
  }
  for (int i = threadIdx.x; i < a.n_zero; i += kThreads) a.zero[i] = 0;
  __syncthreads();
  const double mine = walk_items<false>(a, sm, 0x7fffffff, 0.0, false, &pre);
  double threshold = 0.0;
  int span = 0;  // the first half's steps of a split item (0: half of them)
  if (split) {
    const double avg = block_sum(mine, sm) * a.split_heads / a.slots;  // per compute unit
    if (a.span_pct > 0) {
      span = (int)ceil(avg * a.span_pct / 100.0);
      threshold = span;
    } else {
      threshold = avg / 2.0;
    }
  }
  int total = bucket_starts(sm, threshold, split ? a.max_pairs : 0);
  const int cut = sm.cut;  // > threshold: a split item's halves are non-empty
  if (cut != 0x7fffffff) {  // recount with the heavy items split
    for (int i = threadIdx.x; i < kHistSlots; i += kThreads) sm.hist[i] = 0;
    __syncthreads();
    walk_items<false>(a, sm, cut, span, a.numseqs <= kThreads);
    total = bucket_starts(sm, 0.0, 0);
  }
  walk_items<true>(a, sm, cut, span, a.numseqs <= kThreads);
  for (int i = total + threadIdx.x; i < a.cap; i += kThreads) put_item(a, i, -1, -1, 0, -1);
}

// delta = rowsum(O * dO) and lse * log2(e) for kDeltaPasses * 256 / (D / 8)
// (token, head) rows, D / 8 lanes per row; every pass's loads are issued before
// the first reduction.  The tile loops then form P = exp2(S * scale * log2(e) -
// lse2) with one FMA.
constexpr int kDeltaPasses = 4;

template <int D, bool kGated>
__device__ void delta_block(const DeltaArgs& a, int b) {
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;            // lanes per row
  constexpr int RPP = kThreads / LPR;   // rows per pass
  const int c = threadIdx.x % LPR;
  const int64_t rows = (int64_t)a.T * a.Hq;
  const bool rows32 = rows <= 0x7fffffff;  // (token, head) of a row by a 32-bit division
  bf16x8 ov[kDeltaPasses], dv[kDeltaPasses], gv[kDeltaPasses], lv[kDeltaPasses];
  int t[kDeltaPasses], h[kDeltaPasses];
  bool valid[kDeltaPasses];
  const bool has_lo = a.o_lo != nullptr && (a.lo_gate == nullptr || *a.lo_gate != 0);
#pragma unroll
  for (int i = 0; i < kDeltaPasses; ++i) {
    const int64_t row = ((int64_t)b * kDeltaPasses + i) * RPP + threadIdx.x / LPR;  // row = t * Hq + h
    valid[i] = row < rows;
    t[i] = !valid[i] ? 0 : rows32 ? (int)((uint32_t)row / (uint32_t)a.Hq) : (int)(row / a.Hq);
    h[i] = valid[i] ? (int)(row - (int64_t)t[i] * a.Hq) : 0;
    if (valid[i]) {
      // O, its low half and the gate are read here once, so their loads are
      // non-temporal: dO, which the tile kernels stream next, keeps its place in
      // the caches (backward 1.1-1.6% faster on 8 x 2048 and 64 x 1024 tokens)
      ov[i] = __builtin_nontemporal_load((const bf16x8*)&a.o[(int64_t)t[i] * a.o_st + (int64_t)h[i] * a.o_sh + c * 8]);
      dv[i] = *(const bf16x8*)&a.dout[(int64_t)t[i] * a.do_st + (int64_t)h[i] * a.do_sh + c * 8];
      if constexpr (kGated)
        gv[i] = __builtin_nontemporal_load((const bf16x8*)&a.gate[(int64_t)t[i] * a.g_st + (int64_t)h[i] * a.g_sh + c * 8]);
      lv[i] = has_lo ? __builtin_nontemporal_load(
                           (const bf16x8*)&a.o_lo[(int64_t)t[i] * a.olo_st + (int64_t)h[i] * a.olo_sh + c * 8])
                     : bf16x8{};
    }
  }
#pragma unroll
  for (int i = 0; i < kDeltaPasses; ++i) {
    float acc = 0.f;
    if (valid[i]) {
      if constexpr (kGated) {
        bf16x8 ds, dg;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float s = round_to(sigmoid_bf16((float)gv[i][e]), bf16_t());
          const float dy = (float)dv[i][e], o = (float)ov[i][e];
          const float dso = round_to(dy * s, bf16_t());   // the attention's upstream gradient
          const float dsg = round_to(dy * o, bf16_t());   // gradient of sigmoid(gate)
          ds[e] = (bf16_t)dso;
          dg[e] = (bf16_t)(dsg * (1.0f - s) * s);
          acc += has_lo ? dso * o + dso * (float)lv[i][e] : dso * o;
        }
        *(bf16x8*)&a.dout_s[(int64_t)t[i] * a.ds_st + (int64_t)h[i] * a.ds_sh + c * 8] = ds;
        *(bf16x8*)&a.dgate[(int64_t)t[i] * a.dg_st + (int64_t)h[i] * a.dg_sh + c * 8] = dg;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float dy = (float)dv[i][e];
          acc += has_lo ? (float)ov[i][e] * dy + (float)lv[i][e] * dy : (float)ov[i][e] * dy;
        }
      }
    }
#pragma unroll
    for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (valid[i] && c == 0) {
      a.delta[(int64_t)h[i] * a.T + t[i]] = acc;
      a.lse2[(int64_t)h[i] * a.T + t[i]] = a.lse[(int64_t)h[i] * a.lse_sh + t[i]] * kLog2e;
    }
  }
}

// K magnitude scan: workgroup b sets slot b to 1 if a bf16 element of its share
// of the key rows inside sequences, tokens [cu_seqlens[0], cu_seqlens[numseqs])
// of the [T, Hkv, D] rows, has |k| > the threshold, else to 0.  The
// kKScanSlots * 256 threads take the Hkv * D / 8 sixteen-byte units of a row
// side by side (consecutive threads, consecutive units of a head) and step
// down the rows: the address arithmetic is additions, not a division per
// unit, which bounded the scan by the VALU rather than by HBM.  Padding rows
// are never attended, so whatever they hold cannot change the decision.
// Magnitudes are compared as integers: for finite bf16 the bits with the sign
// cleared order like the values (a NaN compares above any threshold and sets
// the slot).
__device__ void kscan_block(const KScanArgs& a, int b) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  const int upr = a.D / 8;  // 16-byte units per row and head
  int first = a.numseqs > 0 ? a.cu_seqlens[0] : 0;
  int last = a.numseqs > 0 ? a.cu_seqlens[a.numseqs] : 0;
  first = first < 0 ? 0 : (first > a.T ? a.T : first);
  last = last < first ? first : (last > a.T ? a.T : last);
  const int rows = last - first;
  const int row_units = a.Hkv * upr;  // units of one packed row, all kv heads
  constexpr int kScanThreads = kKScanSlots * kThreads;
  u16x2 mx = {0, 0};
  auto fold = [&](i32x4 w) {
#pragma unroll
    for (int e = 0; e < 4; ++e) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2, w[e] & 0x7fff7fff));
  };
  const int t = b * kThreads + threadIdx.x;
  if (row_units <= kScanThreads) {
    // Thread t keeps one unit (kv head, column) of every row_step-th row from
    // row t / row_units on: one division per thread, then additions only.
    const int row_step = kScanThreads / row_units;
    const int r0 = t / row_units;
    if (r0 < row_step) {
      const int cu = t - r0 * row_units;
      const int hk = cu / upr, c = cu - hk * upr;
      const bf16_t* p = a.k + (int64_t)(first + r0) * a.k_st + (int64_t)hk * a.k_sh + c * 8;
      const int64_t pstep = (int64_t)row_step * a.k_st;
      int64_t r = r0;
      for (; r + 3 * row_step < rows; r += 4 * row_step) {  // four loads in flight
        i32x4 w[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = *(const i32x4*)(p + j * pstep);
#pragma unroll
        for (int j = 0; j < 4; ++j) fold(w[j]);
        p += 4 * pstep;
      }
      for (; r < rows; r += row_step) {
        fold(*(const i32x4*)p);
        p += pstep;
      }
    }
  } else {
    // Rows wider than the grid (Hkv * D > 8 * kScanThreads): unit by unit.
    const int64_t units = (int64_t)rows * row_units;
    for (int64_t u = t; u < units; u += kScanThreads) {
      const int64_t row = u / row_units;
      const int cu = (int)(u - row * row_units);
      const int hk = cu / upr, c = cu - hk * upr;
      fold(*(const i32x4*)&a.k[(int64_t)(first + row) * a.k_st + (int64_t)hk * a.k_sh + c * 8]);
    }
  }
  const int over = (uint32_t)mx[0] > a.thr_bits || (uint32_t)mx[1] > a.thr_bits;
  const int any = __syncthreads_or(over);
  if (threadIdx.x == 0) a.slots[b] = any ? 1 : 0;
}

// Zeroes the padding rows of one tensor: the rows t < first or t >= last of
// the packed rows, first = cu_seqlens[0], last = min(cu_seqlens[numseqs],
// total_seqlen).  The fill_blocks workgroups of the target take 16-row chunks
// of those rows in turn, so a batch without padding costs one bounded set of
// workgroups that exit at once, not one per 16 rows of T.
__device__ void fill_block(const FillArgs& a, int b, int fill_blocks) {
  int first = a.numseqs > 0 ? a.cu_seqlens[0] : a.T;
  int last = a.numseqs > 0 ? a.cu_seqlens[a.numseqs] : 0;
  first = first < 0 ? 0 : (first > a.T ? a.T : first);
  if (last > a.total_seqlen) last = a.total_seqlen;
  last = last < first ? first : (last > a.T ? a.T : last);
  const int n_pad = first + (a.T - last);  // padding row j: j < first ? j : last + (j - first)
  const int chunks = a.row_bytes / 4;      // row_bytes is a multiple of 4
  for (int j0 = b * kFillRows; j0 < n_pad; j0 += fill_blocks * kFillRows) {
    for (int i = threadIdx.x; i < kFillRows * a.H * chunks; i += kThreads) {
      const int tt = i / (a.H * chunks);
      const int rem = i % (a.H * chunks);
      const int h = rem / chunks, c = rem % chunks;
      const int j = j0 + tt;
      if (j >= n_pad) continue;
      const int t = j < first ? j : last + (j - first);
      char* row = (char*)a.x + ((int64_t)t * a.st + (int64_t)h * a.sh) * a.elem_bytes;
      ((uint32_t*)row)[c] = 0u;
      if (c == 0 && a.lse != nullptr) a.lse[(int64_t)h * a.lse_sh + t] = -INFINITY;
    }
  }
}

template <int kDeltaD, bool kGated>  // kDeltaD = 0: no delta rows
__global__ __launch_bounds__(kThreads) void prologue_kernel(const PrologueArgs a) {
  int b = blockIdx.x;
  if (b < a.nplan) {
    plan_block(b == 0 ? a.plan[0] : a.plan[1]);
    return;
  }
  b -= a.nplan;
  if (b < a.kscan_blocks) {
    kscan_block(a.kscan, b);
    return;
  }
  b -= a.kscan_blocks;
  if constexpr (kDeltaD > 0) {
    if (b < a.delta_blocks) {
      delta_block<kDeltaD, kGated>(a.delta, b);
      return;
    }
    b -= a.delta_blocks;
  }
  const int target = b / a.fill_blocks;
  fill_block(a.fill[target], b - target * a.fill_blocks, a.fill_blocks);
}

}  // namespace

int plan_capacity(int total_tokens, int numseqs, int /*max_seqlen_all*/) {
  if (numseqs <= 0 || total_tokens <= 0) return 0;
  const int64_t bound = (int64_t)(total_tokens + kPlanTile - 1) / kPlanTile + numseqs;
  return (int)(bound < 0x7fffffff ? bound : 0x7fffffff);
}

KScanArgs kscan_args(const bf16_t* k, int64_t k_st, int64_t k_sh, int T, int Hkv, int D, float scale, int* slots,
                     const int32_t* cu_seqlens, int numseqs) {
  KScanArgs ks;
  ks.k = k; ks.k_st = k_st; ks.k_sh = k_sh;
  ks.T = T; ks.Hkv = Hkv; ks.D = D;
  ks.cu_seqlens = cu_seqlens;
  ks.numseqs = numseqs;
  const float thr = kSplitThreshold / scale;  // as bf16 magnitude bits, rounded toward zero
  uint32_t bits;
  __builtin_memcpy(&bits, &thr, 4);
  ks.thr_bits = (bits >> 16) & 0x7fffu;
  ks.slots = slots;
  return ks;
}

PlanArgs plan_args(const int32_t* cu_seqlens, const int32_t* prefix_lens, int numseqs, int total_seqlen,
                   int is_causal, int total_tokens, int kind, int group, int cap, void* items) {
  PlanArgs a;
  a.cu_seqlens = cu_seqlens;
  a.prefix_lens = prefix_lens;
  a.numseqs = numseqs;
  a.total_seqlen = total_seqlen;
  a.is_causal = is_causal;
  a.T = total_tokens;
  a.kind = kind;
  a.group = group;
  a.cap = cap;
  a.items = items;
  a.split_heads = 0;
  a.max_pairs = 0;
  a.slots = 0;
  a.span_pct = kind == 2 ? 100 : 0;
  a.zero = nullptr;
  a.n_zero = 0;
  return a;
}

BwdWorkspace bwd_workspace_layout(int total_tokens, int num_q_heads, int numseqs, int max_seqlen_all,
                                  size_t dout_bytes, size_t dscore_bytes, int chunk_head_dim) {
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  BwdWorkspace w;
  const size_t rows = (size_t)(total_tokens > 0 ? total_tokens : 0) * (size_t)(num_q_heads > 0 ? num_q_heads : 0);
  w.cap_q = plan_capacity(total_tokens, numseqs, max_seqlen_all);
  const int64_t ph = (int64_t)w.cap_q * (num_q_heads > 0 ? num_q_heads : 0);
  w.pair_heads = (int)(ph < kSplitPairHeads ? ph : kSplitPairHeads);
  w.cap_k = w.cap_q + w.pair_heads;
  w.delta = 0;
  w.lse2 = align(w.delta + rows * sizeof(float));
  w.plan_q = align(w.lse2 + rows * sizeof(float));
  w.plan_k = align(w.plan_q + (size_t)w.cap_q * sizeof(int4));
  w.counters = align(w.plan_k + (size_t)w.cap_k * sizeof(int4));
  w.kscan = align(w.counters + ((size_t)w.pair_heads + kCounterWordsAfterPairs) * sizeof(int));
  w.slots = align(w.kscan + (size_t)kKScanSlots * sizeof(int));
  w.dout = align(w.slots + (size_t)w.pair_heads * 2 * kSplitSlotFloats * sizeof(float));
  w.total = dout_bytes > 0 ? w.dout + dout_bytes : w.slots + (size_t)w.pair_heads * 2 * kSplitSlotFloats * sizeof(float);
  w.dscore = align(w.total);
  if (dscore_bytes > 0) w.total = w.dscore + dscore_bytes;
  w.chunk_slots = chunk_head_dim > 0 && w.cap_q > 0 ? chunk_slots(num_q_heads) : 0;
  w.chunk_list = align(w.total);
  w.chunk_ctr = align(w.chunk_list + (size_t)(w.cap_q + w.chunk_slots) * sizeof(int4));
  w.chunk_part = align(w.chunk_ctr + (size_t)w.chunk_slots * (size_t)(num_q_heads > 0 ? num_q_heads : 0) * sizeof(int));
  if (w.chunk_slots > 0)
    w.total = w.chunk_part + (size_t)w.chunk_slots * (size_t)num_q_heads * chunk_slot_bytes(chunk_head_dim);
  return w;
}

SideStream* side_stream() {
  constexpr int kMaxDevices = 64;
  thread_local SideStream side[kMaxDevices];
  thread_local bool ready[kMaxDevices] = {false};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  if (!ready[dev]) {
    SideStream ss;
    if (hipStreamCreateWithFlags(&ss.stream, hipStreamNonBlocking) != hipSuccess) return nullptr;
    if (hipEventCreateWithFlags(&ss.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&ss.join, hipEventDisableTiming) != hipSuccess)
      return nullptr;
    side[dev] = ss;
    ready[dev] = true;
  }
  return &side[dev];
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 256;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  if (dev < 64) cached[dev] = n;
  return n;
}

FillArgs fill_args(void* x, int64_t st, int64_t sh, float* lse, int64_t lse_sh, const int32_t* cu, int numseqs,
                   int total_seqlen, int T, int H, int D, int elem_bytes) {
  FillArgs a;
  a.x = x; a.st = st; a.sh = sh; a.lse = lse; a.lse_sh = lse_sh; a.cu_seqlens = cu;
  a.numseqs = numseqs; a.total_seqlen = total_seqlen; a.T = T; a.H = H;
  a.row_bytes = D * elem_bytes; a.elem_bytes = elem_bytes;
  return a;
}

hipError_t launch_prologue(const Prologue& pro, hipStream_t stream) {
  PrologueArgs a;
  a.nplan = 0;
  for (int i = 0; i < pro.nplan; ++i)
    if (pro.plan[i].cap > 0) a.plan[a.nplan++] = pro.plan[i];
  a.delta = pro.delta;
  a.kscan = pro.kscan;
  a.kscan_blocks = pro.has_kscan ? kKScanSlots : 0;
  a.delta_blocks = 0;
  int delta_d = 0;
  if (pro.has_delta && (int64_t)pro.delta.T * pro.delta.Hq > 0) {
    delta_d = pro.delta.D;
    const int64_t threads = (int64_t)pro.delta.T * pro.delta.Hq * (delta_d / 8);
    const int64_t per_block = (int64_t)kThreads * kDeltaPasses;
    a.delta_blocks = (int)((threads + per_block - 1) / per_block);
  }
  a.nfill = 0;
  a.fill_blocks = 0;
  for (int i = 0; i < pro.nfill; ++i)
    if (pro.fill[i].T > 0 && pro.fill[i].H > 0) {
      a.fill[a.nfill++] = pro.fill[i];
      // every target has the same T; at most kFillWgs workgroups each
      const int rows = (pro.fill[i].T + kFillRows - 1) / kFillRows;
      a.fill_blocks = rows < kFillWgs ? rows : kFillWgs;
    }
  const int64_t blocks = (int64_t)a.nplan + a.delta_blocks + a.kscan_blocks + (int64_t)a.nfill * a.fill_blocks;
  if (blocks == 0) return hipSuccess;
  const dim3 grid((unsigned)blocks), block(kThreads);
  const bool gated = delta_d > 0 && pro.delta.gate != nullptr;
  void (*kernel)(PrologueArgs) = nullptr;
  switch (delta_d) {
    case 0: kernel = prologue_kernel<0, false>; break;
    case 64: kernel = gated ? prologue_kernel<64, true> : prologue_kernel<64, false>; break;
    case 128: kernel = gated ? prologue_kernel<128, true> : prologue_kernel<128, false>; break;
    default: return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL(kernel, grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
