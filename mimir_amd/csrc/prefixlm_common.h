// Shared device helpers and internal launcher declarations for the gfx950
// prefix-LM attention kernels.  Everything here is CDNA4-specific: wave64,
// bf16 MFMA 32x32x16, buffer resources with hardware range checking,
// ds_read_b64_tr_b16 transposing LDS reads and v_permlane32_swap.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/mimir_prefixlm.h"

namespace mimir {

typedef __bf16 bf16_t;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Compile-time flag for generic lambdas (masked / unmasked tile bodies).
template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Mask algebra.  Inside one sequence with prefix p the reference mask
// (flash_attention_prefixlm_dense.py:61-69) is
//   allowed(i, j) = (i < p && j < p) || (i >= p && j <= i)
// which is exactly j < kend(i) with kend(i) = max(p, i + 1).  is_causal drops the
// prefix (dense.py:61-62), i.e. p = 0.  The column dual is
// qstart(j) = (j < p) ? 0 : j  (flash_attention_prefixlm_mps.py:1147-1149).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int kend_of(int p, int i) { return i + 1 > p ? i + 1 : p; }
__device__ __forceinline__ int qstart_of(int p, int j) { return j < p ? 0 : j; }

// Per-sequence geometry shared by every kernel.
struct SeqGeom {
  int start;  // first packed token of the sequence
  int n;      // keys (sequence length)
  int nq;     // active query rows: rows >= total_seqlen produce zeros
  int p;      // effective prefix length, clamped to [0, n]; 0 when is_causal
};

// Grid x extent for `n` (sequence, head) work columns.  Workgroups are dealt to
// the 8 XCDs round-robin by linear id, so with an even row width every column
// would keep all of its tiles (rows) on one XCD -- whole sequences of heavy
// prefix tiles pile up on half of the XCDs.  An odd width rotates each row by
// one XCD; the padding column exits at once.
inline unsigned xcd_spread_width(int n) { return (unsigned)(n | 1); }
// XCDs of an MI355X in SPX mode: workgroup b of a launch runs on XCD b % kXcds
// (measured: the XCC_ID hardware register of every workgroup).
constexpr int kXcds = 8;

// Sequence bounds are clamped to the packed length T so that malformed metadata
// can never address memory outside the [T, ...] tensors.
// Loads through the constant address space: with a wave-uniform index they
// are scalar loads (the constant cache, one instruction per wave, into scalar
// registers), otherwise ordinary vector loads.  Only for memory no kernel
// running beside the reader writes: the work lists (the prologue's, finished
// before the consumer starts) and the sequence metadata.
template <typename T>
__device__ __forceinline__ T load_const(const T* p, int64_t i) {
  return ((const __attribute__((address_space(4))) T*)p)[i];
}
// A work-list entry, whole, for a whole workgroup (i uniform): one scalar load
// waited for at once (the compiler would otherwise load the first word alone
// for the padding test and the rest behind it).
__device__ __forceinline__ int4 load_entry(const int4* list, int i) {
  const int* w = (const int*)list + 4 * (int64_t)i;
  const int x = load_const(w, 0), y = load_const(w, 1), z = load_const(w, 2), v = load_const(w, 3);
  __asm__ volatile("" ::"s"(x), "s"(y), "s"(z), "s"(v));
  return make_int4(x, y, z, v);
}

// kUniform: s is the same for the whole workgroup; the three loads are then
// scalar loads waited for together, before any branch the compiler could sink
// one of them behind (which costs a kernel another round trip to memory before
// its first tile).
template <bool kUniform = false>
__device__ __forceinline__ SeqGeom load_seq(const int32_t* __restrict__ cu_seqlens,
                                            const int32_t* __restrict__ prefix_lens, int s,
                                            int total_seqlen, int is_causal, int T) {
  SeqGeom g;
  int start, end, p;
  if constexpr (kUniform) {
    // the prefix length is read whether or not it is used, and masked
    start = load_const(cu_seqlens, s);
    end = load_const(cu_seqlens, s + 1);
    const int pl = load_const(prefix_lens, s);
    __asm__ volatile("" ::"s"(start), "s"(end), "s"(pl));
    p = pl & (is_causal ? 0 : -1);
  } else {
    start = cu_seqlens[s];
    end = cu_seqlens[s + 1];
    p = is_causal ? 0 : prefix_lens[s];
  }
  start = start < 0 ? 0 : (start > T ? T : start);
  end = end < start ? start : (end > T ? T : end);
  g.start = start;
  g.n = end - start;
  int nq = total_seqlen - g.start;
  g.nq = nq < 0 ? 0 : (nq > g.n ? g.n : nq);
  g.p = p < 0 ? 0 : (p > g.n ? g.n : p);
  return g;
}

// ---------------------------------------------------------------------------
// Buffer resources.  The descriptor's num_records bounds every access: a load
// whose byte offset falls outside returns zeros, which is how rows beyond the
// end of a sequence are zero-filled without branches.
// ---------------------------------------------------------------------------
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Bytes covering rows [0, rows) of a bf16 matrix with row stride `stride`
// elements whose rows hold `d` values: the num_records of a per-sequence resource.
__device__ __forceinline__ uint32_t rows_bytes(int rows, int64_t stride, int d) {
  return rows > 0 ? (uint32_t)(((int64_t)(rows - 1) * stride + d) * 2) : 0u;
}
// 32-bit form for tiles inside one tensor (the C ABI bounds every span by 2 GiB).
__device__ __forceinline__ uint32_t rows_bytes32(int rows, uint32_t stride, int d) {
  return rows > 0 ? ((uint32_t)(rows - 1) * stride + (uint32_t)d) * 2u : 0u;
}

__device__ __forceinline__ i32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}
__device__ __forceinline__ float buf_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}

// The lane id, formed by instructions the compiler cannot see through: a value
// derived from it is recomputed where it is used instead of being held in a
// register (or spilled) across a loop.
__device__ __forceinline__ int opaque_lane_id() {
  int l;
  __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Pair (x[l % 32], x[l % 32 + 32]) on every lane via v_permlane32_swap, which
// exchanges vdst of lanes 32..63 with vsrc of lanes 0..31.  The two results are
// read through int temporaries: __builtin_bit_cast applied directly to the
// elements of the returned pair yields the first element twice on this compiler.
__device__ __forceinline__ void halves(float x, float& lo, float& hi) {
  const int xi = __float_as_int(x);
  auto r = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  const int a = r[0], b = r[1];
  lo = __int_as_float(a);
  hi = __int_as_float(b);
}
__device__ __forceinline__ float xor32_max(float x) {
  float a, b;
  halves(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float xor32_sum(float x) {
  float a, b;
  halves(x, a, b);
  return a + b;
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Transposing LDS read.  Within each group of 16 lanes, lane j supplies the
// address of 4 consecutive bf16 (row j/4, columns 4*(j%4)..+3 of a 4x16 block);
// lane i receives column i of that block (rows 0..3).
__device__ __forceinline__ bf16x4 lds_read_tr16(const bf16_t* p) {
  i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

__device__ __forceinline__ bf16x8 cat8(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ bf16x8 to_bf16x8(f32x8 v) { return __builtin_convertvector(v, bf16x8); }

// Element-type rounding of an fp32 value (round to nearest even for bf16).
__device__ __forceinline__ float round_to(float x, bf16_t) { return (float)(bf16_t)x; }
__device__ __forceinline__ float round_to(float x, float) { return x; }
// Logistic sigmoid in fp32, 1 / (1 + exp(-x)), the formula torch evaluates
// (in fp32 for bf16 tensors) for torch.sigmoid.
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }
// The same with the hardware exp2 and reciprocal (about 1 ulp each): for values
// that are rounded to bf16 right after, where the difference to sigmoid_f32
// changes a result only when it lies within ~2^-22 of a bf16 rounding boundary.
__device__ __forceinline__ float sigmoid_bf16(float x) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp2(-x * kLog2e));
}

// ---------------------------------------------------------------------------
// Rotary position embedding inside the attention kernels (rotate-half
// convention, src/mimir/model/layers.py:24-40): float32 cos / sin rows [T, D],
// one per token; column d pairs with d + D/2.  A register-resident operand is
// rotated where it is loaded (Q in the forward), and the gradients of the
// rotated operands are mapped back to the unrotated ones where they are stored
// (dQ, dK), with the roundings of prefixlm_layer.hip's rope_kernel:
//   y1  = round(x1 * cos[d] - x2 * sin[d])
//   y2  = round(x2 * cos[d + D/2] + x1 * sin[d + D/2])
//   dx1 = round(round(g1 * cos[d]) + round(g2 * sin[d + D/2]))
//   dx2 = round(round(g2 * cos[d + D/2]) - round(g1 * sin[d]))
// (fp32 products and sums, no contraction; round = to bf16; g the bf16 gradient
// of the rotated operand).
// ---------------------------------------------------------------------------
struct RopeTab {
  const float* cos;  // nullptr: no RoPE
  const float* sin;
  int64_t st;        // elements between the rows of cos / sin
};

// A field of the argument struct at the start of the kernel argument segment
// `seg` (kernel_segment() / uniform_segment()), loaded where it is used: the
// pointer is opaque to the compiler, so the scalar load is not hoisted and the
// value holds no scalar registers across a tile loop (where it would be
// spilled).
template <typename T>
__device__ __forceinline__ T kernarg_at(uint64_t seg, size_t offset) {
  typedef const __attribute__((address_space(4))) char* KPtr;
  KPtr p = (KPtr)seg;
  __asm__ volatile("" : "+s"(p));
  return *(const __attribute__((address_space(4))) T*)(p + offset);
}
// The RoPE tables of the argument struct at `offset`, loaded the same way.
__device__ __forceinline__ RopeTab rope_at(uint64_t seg, size_t offset) {
  return RopeTab{kernarg_at<const float*>(seg, offset + offsetof(RopeTab, cos)),
                 kernarg_at<const float*>(seg, offset + offsetof(RopeTab, sin)),
                 kernarg_at<int64_t>(seg, offset + offsetof(RopeTab, st))};
}

// Rotation of four column pairs (d1 + e, d1 + e + half), e < 4, of token t.
__device__ __forceinline__ void rope_rotate4(const RopeTab& r, int64_t t, int d1, int half, f32x4 x1, f32x4 x2,
                                             bf16x4& y1, bf16x4& y2) {
#pragma clang fp contract(off)
  const float* cr = r.cos + t * r.st;
  const float* sr = r.sin + t * r.st;
  const f32x4 c1 = *(const f32x4*)(cr + d1), c2 = *(const f32x4*)(cr + d1 + half);
  const f32x4 s1 = *(const f32x4*)(sr + d1), s2 = *(const f32x4*)(sr + d1 + half);
  f32x4 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = x1[e] * c1[e] - x2[e] * s1[e];
    b[e] = x2[e] * c2[e] + x1[e] * s2[e];
  }
  y1 = __builtin_convertvector(a, bf16x4);
  y2 = __builtin_convertvector(b, bf16x4);
}

// Gradient of the rotation for four column pairs: g1, g2 hold the bf16-rounded
// gradients of the rotated operand (as fp32 values).
__device__ __forceinline__ void rope_grad4(const RopeTab& r, int64_t t, int d1, int half, f32x4 g1, f32x4 g2,
                                           bf16x4& x1, bf16x4& x2) {
#pragma clang fp contract(off)
  const float* cr = r.cos + t * r.st;
  const float* sr = r.sin + t * r.st;
  const f32x4 c1 = *(const f32x4*)(cr + d1), c2 = *(const f32x4*)(cr + d1 + half);
  const f32x4 s1 = *(const f32x4*)(sr + d1), s2 = *(const f32x4*)(sr + d1 + half);
  f32x4 a, b;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = round_to(g1[e] * c1[e], bf16_t()) + round_to(g2[e] * s2[e], bf16_t());
    b[e] = round_to(g2[e] * c2[e], bf16_t()) - round_to(g1[e] * s1[e], bf16_t());
  }
  x1 = __builtin_convertvector(a, bf16x4);
  x2 = __builtin_convertvector(b, bf16x4);
}

// bf16 rounding of four fp32 values, kept as fp32.
__device__ __forceinline__ f32x4 round4(f32x4 x) {
  return __builtin_convertvector(__builtin_convertvector(x, bf16x4), f32x4);
}

// The bf16 gradient values a lane stores for the columns 32 dt + 8 rg + 4 hi + e
// (e < 4) of one row, from fp32 accumulators acc[dt][4 rg + e] times `scale`:
// the rounded products, or with RoPE (rope.cos set; token t) the gradient of the
// unrotated operand, columns of tiles dt and dt + DT / 2 paired.  put(dt, rg, v)
// receives them.
template <int DT, typename Put>
__device__ __forceinline__ void grad_out(const f32x16 (&acc)[DT], float scale, const RopeTab& rope, int64_t t,
                                         int hi, Put&& put) {
  if (rope.cos == nullptr) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[dt][4 * rg + e] * scale;
        put(dt, rg, __builtin_convertvector(v, bf16x4));
      }
  } else {
#pragma unroll
    for (int dt = 0; dt < DT / 2; ++dt)
#pragma unroll
      for (int rg = 0; rg < 4; ++rg) {
        f32x4 g1, g2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          g1[e] = acc[dt][4 * rg + e] * scale;
          g2[e] = acc[dt + DT / 2][4 * rg + e] * scale;
        }
        bf16x4 x1, x2;
        rope_grad4(rope, t, 32 * dt + 8 * rg + 4 * hi, 16 * DT, round4(g1), round4(g2), x1, x2);
        put(dt, rg, x1);
        put(dt + DT / 2, rg, x2);
      }
  }
}

// ---------------------------------------------------------------------------
// LDS tile layout.  A [64][D] bf16 operand tile is stored with
//   * a row stride of D/8 + 1 sixteen-byte units (one unit of padding), and
//   * logical row k at physical row perm(k), which transposes the 4 x 4 grid
//     of each 16-row block: k = 16 b + 4 i + j -> 16 b + 4 j + i.
// With 64 banks x 4 bytes (16 units), an MFMA operand read serves 16 lanes per
// cycle (16 rows of one block, one unit each) and touches units
// (perm(k) * (D/8 + 1) + c) mod 16: sixteen distinct values.  A transposing
// ds_read_b64_tr_b16 serves 32 lanes per cycle: rows 4i..4i+3 of one block, which
// land on physical rows i, i+4, i+8, i+12, each read at 4 adjacent units -- again
// sixteen distinct units.  Both patterns are therefore conflict-free, and since
// the layout is a row permutation plus padding, every per-k-step / per-d-tile
// displacement is a compile-time constant (an instruction offset).
// ---------------------------------------------------------------------------
template <int D>
struct TileLayout {
  static constexpr int kUnits = D / 8;           // 16-byte units of data per row
  static constexpr int kRowUnits = kUnits + 1;   // with padding
  static constexpr int kRowElems = kRowUnits * 8;
  static constexpr int kElems = 64 * kRowElems;  // one 64-row tile
  // perm is an involution (a 4 x 4 transpose), so unperm == perm
  __device__ static constexpr int perm(int k) { return (k & ~15) | ((k & 3) << 2) | ((k >> 2) & 3); }
  __device__ static constexpr int unperm(int r) { return perm(r); }
  // element offset of (logical row k, column d)
  __device__ static constexpr int off(int k, int d) { return perm(k) * kRowElems + d; }
  // rows x and x + 8 (x < 8) of a block sit two physical rows apart
  static constexpr int kTrSecond = 2 * kRowElems;
};

// Asynchronous global -> LDS copy of 64 consecutive rows of a bf16 matrix (row
// stride `st` elements) into a TileLayout tile, with buffer_load_dwordx4 ... lds.
// One wave instruction writes 64 consecutive 16-byte units of LDS in lane order,
// so the layout is produced on the global side: the lane owning physical unit u
// loads logical row unperm(u / kRowUnits), unit u % kRowUnits; padding units
// read zeros from an out-of-range offset.  The per-lane byte offsets relative to
// the tile's first row never change, so they are computed once; each tile only
// rebuilds the (scalar) buffer resource, whose base is the tile's first row and
// whose size covers the rows still inside the sequence -- rows beyond it read as
// zeros.  The kRowUnits wave instructions of a tile are spread over the NWAVES
// waves, each issued once: kPerWave per wave, or one fewer for the waves
// without a share of the last round (`has_last` false); `rot` picks which
// waves share it, so that two loaders can give their last instructions to
// different waves.  (Repeating the last instruction on the other waves, the
// same data to the same place, kept every wave's count uniform at the cost of
// 7 extra copies per 17 in an 8-wave workgroup: the forward and dK / dV ran
// ~1-2% slower.)  Completion is tracked by vmcnt; callers wait before the
// barrier that publishes the tile, counting each wave's own copies.
template <int D, int NWAVES>
struct TileLoader {
  using L = TileLayout<D>;
  static constexpr int kInst = L::kRowUnits;  // 64 rows * kRowUnits units / 64 lanes
  static constexpr int kPerWave = (kInst + NWAVES - 1) / NWAVES;
  uint32_t voff[kPerWave];
  int lds[kPerWave];  // element offset of each instruction's 1 KiB (wave-uniform)
  int64_t st;
  bool has_last;  // this wave issues an instruction of the last round (wave-uniform)

  // Wave (rot + j) % NWAVES issues instructions j, j + NWAVES, j + 2 NWAVES, ...
  __device__ __forceinline__ TileLoader(int64_t stride, int wave, int lane, int rot = 0) : st(stride) {
    const int wr = (wave + NWAVES - rot) % NWAVES;
    has_last = (kPerWave - 1) * NWAVES + wr < kInst;
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      const int g = min(i * NWAVES + wr, kInst - 1);
      const int u = g * 64 + lane;
      const int prow = u / L::kRowUnits;
      const int c = u - prow * L::kRowUnits;
      const int k = L::unperm(prow);
      voff[i] = c < L::kUnits ? (uint32_t)((k * st + c * 8) * 2) : 0x80000000u;
      lds[i] = g * 512;
    }
  }
  // Copy rows [row0, row0 + 64) of the matrix at `base`; rows >= nrows read as 0.
  __device__ __forceinline__ void issue(const bf16_t* base, int row0, int nrows, bf16_t* tile) const {
    issue_at(base + (int64_t)row0 * st, rows_bytes(nrows - row0, st, D), tile);
  }
  // Same, from the first row's address and the byte size of the rows left.
  __device__ __forceinline__ void issue_at(const bf16_t* first_row, uint32_t bytes, bf16_t* tile) const {
    const __amdgpu_buffer_rsrc_t r = make_rsrc(first_row, bytes);
#pragma unroll
    for (int i = 0; i < kPerWave; ++i) {
      if (i == kPerWave - 1 && !has_last) break;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(tile + lds[i]), 16,
                                               voff[i], 0, 0, 0);
    }
  }
};

// Lane geometry of the operand reads from a TileLayout tile.
//  * MFMA 32x32x16 operand with rows on lanes (A of K Q^T, Q K^T, ...): lane
//    reads logical row 32*mt + (lane & 31), columns 16*ks + 8*(lane >> 5) .. +7:
//    element offset op_base + mt * 32 * kRowElems + ks * 16.
//  * transposed operand (ds_read_b64_tr_b16) over rows 16*kk + 4*(lane >> 5) +
//    0..3 (and + 8), columns 32*dt + 16*((lane >> 4) & 1) + 0..15: element offset
//    tr_base + kk * 16 * kRowElems + dt * 32 (+ kTrSecond for the second read).
template <int D>
struct TileLanes {
  using L = TileLayout<D>;
  int op_base;
  int tr_base;
  __device__ explicit TileLanes(int lane) {
    op_base = L::off(lane & 31, 8 * (lane >> 5));
    const int tj = lane & 15, tg = lane >> 4;
    tr_base = L::off(4 * (tg >> 1) + (tj >> 2), 16 * (tg & 1) + 4 * (tj & 3));
  }
};

// s_waitcnt vmcnt(0) (GFX9 encoding: expcnt and lgkmcnt left at their maxima).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// s_waitcnt lgkmcnt(0) (vmcnt and expcnt left at their maxima).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Wait until at most N vector-memory operations of this wave are outstanding
// (they complete in issue order, so everything older than the last N is done).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate (low field)");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Barrier of a multi-stage LDS pipeline: this wave's LDS reads are complete and
// at most N of its vector-memory operations (the newest tile copies) are still
// in flight, then all waves meet.  Unlike __syncthreads(), whose workgroup
// release fence makes the compiler wait for every outstanding buffer -> LDS
// copy (vmcnt(0)), the tiles issued for later stages stay in flight across it.
// The empty asm statements keep the compiler from moving memory accesses
// across the barrier.
template <int N>
__device__ __forceinline__ void stage_barrier() {
  static_assert(N >= 0 && N < 16, "vmcnt immediate (low field)");
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0070 | N);  // vmcnt(N) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

}  // namespace mimir

namespace mimir {
// The per-call work in front of the tile loops (prefixlm_prologue.hip), run as
// one launch: tile work lists, the backward's delta rows, padding-row fills.
//
// Tile work lists: kind 0 holds 128-row query tiles (forward, dQ) as int2
// (sequence, tile); kind 1 holds 128-key tiles (dK / dV) as int4 (sequence,
// tile, part, pair).  A list is sorted by cost, descending, and padded with
// sequence -1; workgroup r * H + h of a consumer takes entry r for head h.
//
// Kind-1 items may be split: part 0 is a whole key tile; parts 1 and 2 are its
// first and second half of the (q head, 64-query tile) steps, each adding into
// dK / dV of the same keys.  Both halves write fp32 partials to the split slots
// of pair `pair` and the later of the two (per kv head) adds them and stores
// dK / dV (see SplitSlots).  Splitting evens out the workgroups when a few
// heavy key tiles (the prefix tiles, which every query attends) dominate.
constexpr int kPlanTile = 128;
// List entries for any packing of total_tokens tokens into numseqs sequences:
// sum_s ceil(n_s / 128) <= ceil(T / 128) + numseqs.  max_seqlen_all is not used,
// so metadata with an understated max_seqlen_all still lists every tile.
int plan_capacity(int total_tokens, int numseqs, int max_seqlen_all);


struct PlanArgs {
  const int32_t* cu_seqlens;
  const int32_t* prefix_lens;
  int numseqs, total_seqlen, is_causal, T, kind, group, cap;
  void* items;     // int2 [cap] (kind 0) or int4 [cap] (kinds 1 and 2)
  // kind 2 (the forward's query tiles, int4 (sequence, tile, part | parts << 8 |
  // span << 16, chunk slot)): when the grid is small (items * split_heads <
  // slots) the key range of every item costing more than span = ceil(total cost
  // * split_heads / slots) key tiles (at least kChunkMinCost) is cut into parts,
  // at most kChunkMax: the last parts span tiles each, the first the rest;
  // max_pairs (the chunk slots available) = 0 disables it.
  // kind 1: split items costing more than (total cost * split_heads / slots) / 2,
  // heaviest first and whole cost buckets at a time, up to max_pairs items;
  // split_heads = 0 disables splitting.
  int split_heads, max_pairs, slots;
  // kind 2: the part span in percent of the per-slot average (>= 100, so that the
  // parts stay within max_pairs); kind 1: a split item's first half in percent of
  // the per-CU average (0: half its steps)
  int span_pct;
  int* zero;  // n_zero int32 set to 0 (the consumer's counters)
  int n_zero;
};

// Split partials of the dK / dV kernel: per (pair, kv head) one arrival counter
// and two slots (one per part) of fp32 dK then dV, 128 keys x 128 columns each.
// Two more counters after them drive its work queue (next unit, finished
// workgroups).
constexpr int kSplitPairHeads = 384;              // most (pair, kv head) combinations per call
constexpr int kSplitSlotFloats = 2 * 128 * 128;   // dK + dV partial of one part

// Device-side choice of the split products (MimirSplitMode).  The forward's
// prologue (and the backward's DELTA stage when no forward decision is given)
// scans K in kKScanSlots workgroups; slot b is 1 if its share holds an element
// with softmax_scale * |k| > kSplitThreshold.  With AUTO the kernels carry P
// (forward) and dS (backward) as bf16 hi + lo when any slot is set; the forward
// records that decision in a one-word flag the backward reads.  The backward's counter words after the
// split counters and the work queue hold one more flag: non-zero when the dK / dV
// kernel could not store a score-gradient tile (a sequence longer than
// max_seqlen_all), so that the recomputing dQ kernel takes over from the hand-off.
constexpr int kKScanSlots = 512;

// Key-range chunks of the query-tile lists (kind 2: the forward and dQ): small
// grids leave most CUs idle while the heaviest query tiles run, so their key
// ranges are cut into parts that run as separate workgroups and are merged by
// the last to finish.
constexpr int kChunkMax = 16;        // parts per query tile
constexpr int kChunkMinCost = 4;     // key tiles per part, at least
constexpr int kChunkWgs = 512;       // query-tile workgroups resident at once (2 per CU)
constexpr int kChunkHeadSlots = 2 * kChunkWgs;  // chunk slots x q heads, at most
// Chunk slots for Hq heads: with parts cut at the per-workgroup average cost
// of one round, the parts of the split tiles number at most 2 * kChunkWgs / Hq.
inline int chunk_slots(int hq) { return hq > 0 ? kChunkHeadSlots / hq : 0; }
// One chunk slot per (part, q head): the part's fp32 accumulator (O^T or dQ^T;
// per wave DT * 4 float4 per lane, lane-major) then, for the forward, its
// running max and sum per lane.
__host__ __device__ inline size_t chunk_slot_bytes(int d) { return (size_t)4 * (size_t)d * 128 + (size_t)4 * 64 * 8; }
// Whether the grid of a kind-2 list can be small (chunks may be planned), from
// the active tokens n = min(T, total_seqlen): a packing of n tokens has at least
// ceil(n / 128) query tiles when its sequences start at cu_seqlens[0] = 0 (the
// reference's metadata), so the grid can be small only if that many times Hq
// stays below kChunkWgs.  Other metadata (leading padding rows) can have fewer
// tiles; such a call may get no chunk room and then runs uncut: slower, with
// the same results.
inline bool chunk_grid_can_be_small(int total_tokens, int total_seqlen, int hq) {
  const int n = total_seqlen < total_tokens ? total_seqlen : total_tokens;
  return n > 0 && hq > 0 && ((int64_t)n + 127) / 128 * hq < kChunkWgs;
}
// Forward workspace, 256-byte aligned sections: the work list (int4 [cap +
// chunk slots]), the kKScanSlots int32 slots of the K scan, then with chunking
// one arrival counter per (chunk slot, q head) and the chunk slots.
struct FwdWorkspace {
  size_t list, kscan, ctr, part, total;
  int list_cap, chunk_slots;
};
inline FwdWorkspace fwd_workspace_layout(int cap, int hq, int d, bool chunks) {
  auto align = [](size_t x) { return (x + 255) & ~(size_t)255; };
  FwdWorkspace w;
  w.chunk_slots = chunks && cap > 0 ? chunk_slots(hq) : 0;
  w.list_cap = cap > 0 ? cap + w.chunk_slots : 0;
  w.list = 0;
  w.kscan = align((size_t)w.list_cap * 16);
  w.ctr = align(w.kscan + (size_t)kKScanSlots * sizeof(int));
  w.part = align(w.ctr + (size_t)w.chunk_slots * (size_t)(hq > 0 ? hq : 0) * sizeof(int));
  w.total = w.chunk_slots > 0 ? w.part + (size_t)w.chunk_slots * (size_t)hq * chunk_slot_bytes(d)
                              : w.ctr;
  return w;
}
constexpr float kSplitThreshold = 0.75f;
constexpr int kCounterWordsAfterPairs = 3;  // work queue next / finished, dS-incomplete flag

// Backward workspace sections (byte offsets, 256-byte aligned).
// `dout_bytes`: the gated backward's upstream-gradient buffer (0 without a gate).
// Backward workspace; with chunk_head_dim > 0 it ends with the dQ list's
// key-range chunks: that list (int4 [cap_q + chunk slots]), one arrival counter
// per (chunk slot, q head) and the chunk slots (chunk_slot_bytes(head_dim)).
struct BwdWorkspace {
  size_t delta, lse2, plan_q, plan_k, counters, kscan, slots, dout, dscore, chunk_list, chunk_ctr, chunk_part, total;
  int cap_q, cap_k, pair_heads, chunk_slots;
};
BwdWorkspace bwd_workspace_layout(int total_tokens, int num_q_heads, int numseqs, int max_seqlen_all,
                                  size_t dout_bytes = 0, size_t dscore_bytes = 0, int chunk_head_dim = 0);
// head_dim of the dQ list's key-range chunks for these parameters, 0: none.
inline int bwd_chunk_head_dim(const MimirPrefixLMBwdParams& p) {
  return p.dq_key_chunks != 0 && p.dtype == MIMIR_DTYPE_BFLOAT16 && p.head_dim > 0 &&
                 chunk_grid_can_be_small(p.total_tokens, p.total_seqlen, p.num_q_heads)
             ? p.head_dim
             : 0;
}

// Score-gradient hand-off from the dK / dV stage to the dQ stage: bf16 dS in
// blocks of 32 queries x 32 keys (2 KiB), block index (h * rows + row) * width +
// key / 32 with row = floor(start / 32) + s + query / 32 for sequence s starting
// at packed token `start`.  Rows of consecutive sequences never overlap
// (floor(start / 32) + ceil(n / 32) <= floor((start + n) / 32) + 1), so
// rows = floor(T / 32) + numseqs + 1 and width = ceil(max_seqlen / 32) bound
// every block of well-formed metadata.
//
// Inside a block the 32 queries sit at positions in the order the MFMA
// accumulator of the dK / dV kernel leaves them -- position 16 a + 8 b + 4 c + e
// is query 16 a + 8 c + 4 b + e (bits 2 and 3 swapped) -- and (key k, position
// n) at byte (n / 16) * 1024 + k * 32 + (n % 16) * 2: two 1 KiB halves of
// 32 key rows x 16 positions.
constexpr int kDsBlock = 32;
constexpr int kDsBlockElems = kDsBlock * kDsBlock;
struct DscoreGeom {
  int rows, width;
  size_t bytes;
};
inline DscoreGeom dscore_geometry(int total_tokens, int num_q_heads, int numseqs, int max_seqlen_all) {
  DscoreGeom g;
  g.rows = total_tokens / kDsBlock + (numseqs > 0 ? numseqs : 0) + 1;
  g.width = ((max_seqlen_all > 0 ? max_seqlen_all : 0) + kDsBlock - 1) / kDsBlock;
  g.bytes = (size_t)(num_q_heads > 0 ? num_q_heads : 0) * (size_t)g.rows * (size_t)g.width * kDsBlockElems * 2;
  return g;
}
// The position <-> query map of a block row (an involution).
__host__ __device__ constexpr int ds_query_of(int pos) { return (pos & ~12) | ((pos & 4) << 1) | ((pos & 8) >> 1); }

// delta[h, t] = sum_d O[t, h, d] * dO[t, h, d] and lse2[h, t] = lse[h, t] * log2(e), bf16 O / dO.
// With a gate, `dout` is the gradient of the gated output: the rows also form
// the attention's upstream gradient dout_s = round(dout * s) (which delta then
// uses) and dgate = round(round(dout * O) * (1 - s) * s), s = round(sigmoid(gate)).
struct DeltaArgs {
  const bf16_t* o;
  const bf16_t* o_lo;  // optional low half of O (delta from O + O_lo) ...
  const int* lo_gate;  // ... read only if this flag (the forward's split decision) is set; NULL: always
  int64_t olo_st, olo_sh;
  const bf16_t* dout;
  const float* lse;
  float* delta;
  float* lse2;
  int64_t o_st, o_sh, do_st, do_sh, lse_sh;
  int T, Hq, D;
  const bf16_t* gate;  // NULL: no gate
  bf16_t* dgate;
  bf16_t* dout_s;
  int64_t g_st, g_sh, dg_st, dg_sh, ds_st, ds_sh;
};

// Zero the rows of one [T, H, D] tensor (and lse = -inf if non-NULL) that lie
// outside [cu_seqlens[0], min(cu_seqlens[numseqs], total_seqlen)).
struct FillArgs {
  void* x;         // [T, H, D] of elem_bytes
  int64_t st, sh;  // strides in elements
  float* lse;      // optional [H, T]
  int64_t lse_sh;
  const int32_t* cu_seqlens;
  int numseqs, total_seqlen, T, H, row_bytes, elem_bytes;
};

// K magnitude scan for the dQ split decision (see kKScanSlots): kKScanSlots
// workgroups, each over a strided share of the [T, Hkv, D] rows of the tokens
// inside sequences, [cu_seqlens[0], cu_seqlens[numseqs]).
struct KScanArgs {
  const bf16_t* k;
  int64_t k_st, k_sh;
  int T, Hkv, D;
  uint32_t thr_bits;  // bf16 magnitude bits of kSplitThreshold / softmax_scale
  int* slots;         // [kKScanSlots]
  const int32_t* cu_seqlens;
  int numseqs;
};

KScanArgs kscan_args(const bf16_t* k, int64_t k_st, int64_t k_sh, int T, int Hkv, int D, float scale, int* slots,
                     const int32_t* cu_seqlens, int numseqs);

// Whether a kernel splits its bf16 operand (wave-uniform): always, never, or
// (AUTO) as the recorded decision `flag` says, or without one when the K scan
// of this call set any slot.
__device__ __forceinline__ bool split_decision(int mode, const int* slots, const int* flag, int lane) {
  static_assert(kKScanSlots == 2 * 64 * 4, "two int4 loads per lane cover the slots");
  if (mode == MIMIR_SPLIT_ALWAYS) return true;
  if (mode != MIMIR_SPLIT_AUTO) return false;
  if (flag != nullptr) return __builtin_amdgcn_readfirstlane(*flag) != 0;
  const i32x4 a = ((const i32x4*)slots)[lane], b = ((const i32x4*)slots)[lane + 64];
  const int any = (a[0] | a[1] | a[2] | a[3] | b[0] | b[1] | b[2] | b[3]) != 0;
  return __builtin_amdgcn_ballot_w64(any) != 0;
}

// The running kernel's argument segment as an integer.  A function the kernel
// calls gets it as an argument (outside a kernel the segment-pointer builtin
// reads as null) and passes it through uniform_segment(), which puts it back in
// scalar registers; segment_args() then reads the struct at its start through a
// constant-space pointer, with scalar loads as the kernel does.
__device__ __forceinline__ uint64_t kernel_segment() {
  return (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
}
__device__ __forceinline__ uint64_t uniform_segment(uint64_t seg) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)seg);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(seg >> 32));
  return ((uint64_t)hi << 32) | lo;
}
template <typename Args>
__device__ __forceinline__ const Args& segment_args(uint64_t seg) {
  return *(const Args*)(const __attribute__((address_space(4))) Args*)seg;
}

// bf16 hi + lo halves of 8 fp32 values: hi = round(x), lo = round(x - hi).
__device__ __forceinline__ bf16x8 lo_half(f32x8 x, bf16x8 hi) {
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] -= (float)hi[e];
  return __builtin_convertvector(x, bf16x8);
}

struct Prologue {
  PlanArgs plan[2];
  int nplan = 0;
  DeltaArgs delta;
  int has_delta = 0;
  KScanArgs kscan;
  int has_kscan = 0;
  FillArgs fill[3];  // targets of one launch share T
  int nfill = 0;
};

PlanArgs plan_args(const int32_t* cu_seqlens, const int32_t* prefix_lens, int numseqs, int total_seqlen,
                   int is_causal, int total_tokens, int kind, int group, int cap, void* items);
// Compute units of the current device (cached per device).
int device_cu_count();

// A second stream of the current device with fork / join events (created once
// per host thread and device, default priority), or nullptr if that failed.
struct SideStream {
  hipStream_t stream;
  hipEvent_t fork, join;
};
SideStream* side_stream();
FillArgs fill_args(void* x, int64_t st, int64_t sh, float* lse, int64_t lse_sh, const int32_t* cu, int numseqs,
                   int total_seqlen, int T, int H, int D, int elem_bytes);
hipError_t launch_prologue(const Prologue& pro, hipStream_t stream);

// KV-cache attention (prefixlm_cache_bf16.hip): the key split and its workspace.
struct CacheSplit {
  bool decode;     // at most 32 query rows per kv head: the decode kernel
  int n_rt, splits;
  int64_t groups;  // (batch row, kv head, row tile) triples
  int64_t units;   // groups * splits workgroups
  size_t workspace_bytes;
};
CacheSplit cache_split(const MimirCacheAttnParams& p);
hipError_t launch_cache_attn_bf16(const MimirCacheAttnParams& p, hipStream_t stream);

// Layer kernels (prefixlm_layer.hip).
hipError_t launch_rope(const MimirRopeParams& p, hipStream_t stream);
hipError_t launch_gate_fwd_f32(const MimirPrefixLMFwdParams& p, hipStream_t stream);
// float32 gate backward rows: dout_s = dout * s, delta, dgate (one thread per row).
hipError_t launch_gate_bwd_f32(const MimirPrefixLMBwdParams& p, float* dout_s, float* delta, hipStream_t stream);
}  // namespace mimir

namespace mimir {
// Sets the thread-local message mimir_prefixlm_last_error() returns; returns `code`.
int fail_with(int code, const std::string& msg);
}  // namespace mimir

// Internal launchers (implemented per kernel file, dispatched from prefixlm_capi.hip).
// The bf16 launchers add their tile lists (and the backward its delta rows) to
// `pro`, which holds the caller's padding fills, and launch it before their
// tile kernels.
hipError_t mimir_launch_fwd_bf16(const MimirPrefixLMFwdParams& p, mimir::Prologue pro, hipStream_t stream);
hipError_t mimir_launch_bwd_bf16(const MimirPrefixLMBwdParams& p, mimir::Prologue pro, hipStream_t stream,
                                 int stages);
hipError_t mimir_launch_fwd_f32(const MimirPrefixLMFwdParams& p, hipStream_t stream);
hipError_t mimir_launch_bwd_f32(const MimirPrefixLMBwdParams& p, hipStream_t stream, int stages);
bool mimir_bf16_head_dim_supported(int d);
bool mimir_f32_head_dim_supported(int d);
