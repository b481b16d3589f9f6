// Tile work lists for the bf16 kernels: which (sequence, 128-row tile) each
// workgroup takes, heaviest first.
//
// The grids of the forward, dQ and dK/dV kernels used to be (column, tile row)
// rectangles dispatched row by row, which only approximates heaviest-first: on
// batches of a few 2k sequences the last workgroups to start were still large
// and the kernels ended on long tails.  One workgroup of this kernel instead
// computes every item's cost from the metadata on the device (no host copy of
// cu_seqlens / prefix_lens), counting-sorts the items by cost, descending, into
// a list in the caller's workspace, and pads the list with (-1, -1).  Workgroup
// r * H + h of the consumer then takes list entry r for head h: the H heads of
// one item run back to back and the dispatch order is longest-processing-time
// first.  The order inside one cost bucket follows LDS atomics and may differ
// from call to call; every item writes its own outputs, so results do not.
//
// Costs, in 64-row tiles of the inner loop:
//   query tiles (forward, dQ):  key tiles up to kend of the tile's last row,
//                               ceil(max(p, min(m0 + 128, nq)) / 64)
//   key tiles (dK / dV):        G * query tiles from qstart(first key),
//                               G * ceil((nq - qstart(kb0)) / 64), 0 if none
#include "prefixlm_common.h"

namespace mimir {
namespace {

constexpr int kPlanThreads = 1024;
constexpr int kPlanBuckets = 4096;  // costs above kPlanBuckets - 1 share the last bucket
constexpr int kTile = 128;

struct PlanArgs {
  const int32_t* cu_seqlens;
  const int32_t* prefix_lens;
  int numseqs, total_seqlen, is_causal, T, kind, group, cap;
  int2* items;
};

__device__ __forceinline__ int item_count(const SeqGeom& g, int kind) {
  return ((kind == 0 ? g.nq : g.n) + kTile - 1) / kTile;
}

__device__ __forceinline__ int item_cost(const SeqGeom& g, int kind, int group, int t) {
  int c;
  if (kind == 0) {
    const int kend = max(g.p, min(t * kTile + kTile, g.nq));
    c = (kend + 63) / 64;
  } else {
    const int q0 = qstart_of(g.p, t * kTile);
    c = g.nq > q0 ? group * ((g.nq - q0 + 63) / 64) : 0;
  }
  return min(c, kPlanBuckets - 1);
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const PlanArgs a) {
  __shared__ int hist[kPlanBuckets];
  __shared__ int part[kPlanThreads];
  const int tid = threadIdx.x;
  for (int i = tid; i < kPlanBuckets; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  for (int s = tid; s < a.numseqs; s += kPlanThreads) {
    const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
    const int nt = item_count(g, a.kind);
    for (int t = 0; t < nt; ++t) atomicAdd(&hist[item_cost(g, a.kind, a.group, t)], 1);
  }
  __syncthreads();
  // Exclusive scan in descending cost order: bucket c starts after all items of
  // cost > c.  Thread i owns buckets kPlanBuckets-1-4i .. kPlanBuckets-4-4i.
  constexpr int kPer = kPlanBuckets / kPlanThreads;
  int local = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) local += hist[kPlanBuckets - 1 - (kPer * tid + j)];
  part[tid] = local;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {  // inclusive Hillis-Steele scan
    const int v = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  const int total = part[kPlanThreads - 1];
  int run = part[tid] - local;  // exclusive prefix of this thread's buckets
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int b = kPlanBuckets - 1 - (kPer * tid + j);
    const int h = hist[b];
    hist[b] = run;  // becomes the next free position of bucket b
    run += h;
  }
  __syncthreads();
  for (int s = tid; s < a.numseqs; s += kPlanThreads) {
    const SeqGeom g = load_seq(a.cu_seqlens, a.prefix_lens, s, a.total_seqlen, a.is_causal, a.T);
    const int nt = item_count(g, a.kind);
    for (int t = 0; t < nt; ++t) {
      const int pos = atomicAdd(&hist[item_cost(g, a.kind, a.group, t)], 1);
      if (pos < a.cap) a.items[pos] = make_int2(s, t);
    }
  }
  for (int i = total + tid; i < a.cap; i += kPlanThreads) a.items[i] = make_int2(-1, -1);
}

}  // namespace

int plan_capacity(int total_tokens, int numseqs, int max_seqlen_all) {
  if (numseqs <= 0 || max_seqlen_all <= 0) return 0;
  const int64_t rect = (int64_t)numseqs * ((max_seqlen_all + kTile - 1) / kTile);
  const int64_t bound = (int64_t)(total_tokens + kTile - 1) / kTile + numseqs;
  return (int)(rect < bound ? rect : bound);
}

hipError_t launch_plan(const int32_t* cu_seqlens, const int32_t* prefix_lens, int numseqs, int total_seqlen,
                       int is_causal, int total_tokens, int kind, int group, int cap, int2* items,
                       hipStream_t stream) {
  if (cap <= 0) return hipSuccess;
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
  hipLaunchKernelGGL(plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mimir
