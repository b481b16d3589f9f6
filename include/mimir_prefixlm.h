/*
 * mimir_prefixlm.h -- C ABI of the MI355X (gfx950) prefix-LM attention library
 * (libmimir_prefixlm.so).
 *
 * Prefix-LM attention over packed variable-length sequences: inside sequence s
 * (tokens cu_seqlens[s] .. cu_seqlens[s+1]) with prefix length p = prefix_lens[s],
 * local query i may attend local key j iff
 *
 *     j < kend(i),   kend(i) = max(p, i + 1)        (is_causal == 0)
 *     j < i + 1                                    (is_causal != 0)
 *
 * i.e. bidirectional inside the prefix and causal after it
 * (reference: src/mimir/model/flash_attention_prefixlm_dense.py:61-69 and the
 * Metal predicate src/mimir/model/flash_attention_prefixlm_mps.py:43-51).
 *
 * Layout: q [T, Hq, D], k/v [T, Hkv, D], out [T, Hq, D]; every tensor has a
 * unit stride on the last (head_dim) axis and arbitrary token / head strides
 * given in ELEMENTS.  v may therefore be the strided split of a fused
 * gate/q/k/v projection (reference: src/mimir/model/layers.py:183-184).
 * lse is float32 [Hq, T] (natural log of the softmax denominator, scale
 * included), the FlashAttention varlen convention used by
 * src/mimir/model/flash_attention_prefixlm_v2.py:159-160.
 * GQA: query head h reads kv head h / (Hq / Hkv)
 * (reference: flash_attention_prefixlm_dense.py:10-16, repeat_interleave).
 *
 * Query rows >= total_seqlen and rows outside every sequence produce O = 0,
 * lse = -inf and zero dQ (reference: flash_attention_prefixlm_dense.py:43,79-80;
 * flash_attention_prefixlm_v2.py:143,224-226).
 *
 * All device pointers are plain HIP device addresses; `stream` is a hipStream_t
 * (passed as void* so that this header needs no HIP include).  Every entry point
 * only enqueues work on `stream` and never synchronises it.  Status 0 is success;
 * on failure mimir_prefixlm_last_error() returns a thread-local message.
 */
#ifndef MIMIR_PREFIXLM_H
#define MIMIR_PREFIXLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MIMIR_PREFIXLM_ABI_VERSION 8

/* Element types of q/k/v/out/dout/dq/dk/dv (lse and the workspace are float32). */
enum MimirDType {
  MIMIR_DTYPE_FLOAT32 = 0,
  MIMIR_DTYPE_BFLOAT16 = 1
};

/* Status codes.  The Python binding maps them to the exception types the
 * reference raises for the same conditions. */
enum MimirStatus {
  MIMIR_OK = 0,
  MIMIR_ERR_INVALID_ARGUMENT = 1, /* ValueError  (dense.py:14,54-55; fa4.py:437,460,505) */
  MIMIR_ERR_UNSUPPORTED_DTYPE = 2,/* TypeError   (mps.py:1390-1391) */
  MIMIR_ERR_UNSUPPORTED_SHAPE = 3,/* ValueError: head_dim / size not supported by the kernels */
  MIMIR_ERR_HIP = 4               /* RuntimeError: a HIP launch or runtime call failed */
};

typedef struct MimirPrefixLMFwdParams {
  const void* q;              /* [T, Hq, D]  */
  const void* k;              /* [T, Hkv, D] */
  const void* v;              /* [T, Hkv, D] */
  void* out;                  /* [T, Hq, D], written for every row 0..T-1 */
  float* lse;                 /* [Hq, T] float32, may be NULL */
  const int32_t* prefix_lens; /* device int32 [>= numseqs]     */
  const int32_t* causal_lens; /* device int32 [>= numseqs]     (only read by mimir_prefixlm_check_metadata) */
  const int32_t* cu_seqlens;  /* device int32 [>= numseqs + 1] */
  int64_t q_stride_token, q_stride_head;
  int64_t k_stride_token, k_stride_head;
  int64_t v_stride_token, v_stride_head;
  int64_t out_stride_token, out_stride_head;
  int64_t lse_stride_head;    /* lse[h * lse_stride_head + t] */
  int32_t total_tokens;       /* T = q.shape[0] */
  int32_t num_q_heads;        /* Hq */
  int32_t num_kv_heads;       /* Hkv, Hq % Hkv == 0 */
  int32_t head_dim;           /* D */
  int32_t numseqs;
  int32_t total_seqlen;
  int32_t max_seqlen_all;     /* upper bound of cu_seqlens[s+1] - cu_seqlens[s] */
  int32_t is_causal;
  int32_t dtype;              /* enum MimirDType */
  float softmax_scale;        /* > 0; the reference uses 1/sqrt(D) */
  void* workspace;            /* device memory, >= mimir_prefixlm_fwd_workspace_bytes(); 16-byte aligned */
  size_t workspace_bytes;
  /* Optional sigmoid output gate (NULL: none).  With a gate the forward also
   * writes gated_out = sigmoid(gate) * out, rounded as the reference's
   * torch.sigmoid(gate) * attn_output in the element type
   * (src/mimir/model/layers.py:239): s = round(sigmoid(gate)), then
   * round(s * round(attention)).  out keeps the ungated attention output, which
   * the backward needs. */
  const void* gate;           /* [T, Hq, D] */
  int64_t gate_stride_token, gate_stride_head;
  void* gated_out;            /* [T, Hq, D]; required with a gate */
  int64_t gated_out_stride_token, gated_out_stride_head;
  /* Optional low half of the output (NULL: not written; bf16 only): out_lo =
   * round(O - round(O)) with O the float32 attention output, so out + out_lo
   * carries ~16 significant bits.  The backward's delta = rowsum(dout * O) reads
   * it (MimirPrefixLMBwdParams.out_lo); with bf16 O alone that row sum carries
   * the output's rounding into every dS of the row.  No reference counterpart. */
  void* out_lo;               /* [T, Hq, D] */
  int64_t out_lo_stride_token, out_lo_stride_head;
  int32_t split_mode;         /* enum MimirSplitMode (bf16; P in O = P V) */
  /* Optional (NULL: none): the forward writes its split decision (0 / 1) here,
   * and then writes out_lo only when it splits.  Passed to the backward
   * (MimirPrefixLMBwdParams.split_flag), the backward follows the same decision
   * without scanning K again and reads out_lo only when it is set. */
  int32_t* split_flag;        /* device int32 [1] */
  /* Optional rotary position embedding of q inside the kernel (bf16 only;
   * rope_cos NULL: none), replacing the apply_rotary_pos_emb of q before the
   * attention call (src/mimir/model/layers.py:186-189, rotate-half convention
   * layers.py:24-40): q is then the unrotated query, rotated where the kernel
   * loads it, with the roundings of mimir_prefixlm_rope; k must already be the
   * rotated key (mimir_prefixlm_rope: the kernel streams K through LDS).  With
   * q_rope non-NULL the kernel also writes the rotated q there (the rows below
   * total_seqlen of every sequence), the q operand of the backward. */
  const float* rope_cos;      /* [T, D] float32, 16-byte aligned rows */
  const float* rope_sin;      /* [T, D] float32 */
  int64_t rope_stride_token;  /* elements between rows of rope_cos / rope_sin (multiple of 4) */
  void* q_rope;               /* optional out [T, Hq, D] */
  int64_t q_rope_stride_token, q_rope_stride_head;
} MimirPrefixLMFwdParams;

/* Whether the bf16 kernels carry the softmax probabilities P and the score
 * gradients dS as two bf16 halves.  A bf16 MFMA operand keeps 8 significant
 * bits; split, the operand is hi + lo with lo = round(x - hi) and every product
 * with it takes one more MFMA (forward O = P V, backward dK = dS^T Q and
 * dQ = dS K), which removes that rounding from the result.  dQ and dK are sums
 * of cancelling terms (every row of dS sums to zero) and delta = rowsum(dout * O)
 * inherits the rounding of O, so with large key or query entries these roundings
 * dominate the gradients' error.  AUTO splits when softmax_scale * max|K| > 0.75
 * anywhere in the call: the prologue of the forward and of the backward's DELTA
 * stage scans K on the device, and the kernels read the result (no host
 * synchronisation).  No reference counterpart. */
enum MimirSplitMode {
  MIMIR_SPLIT_AUTO = 0,
  MIMIR_SPLIT_ALWAYS = 1,
  MIMIR_SPLIT_NEVER = 2
};

typedef struct MimirPrefixLMBwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* out;            /* forward output [T, Hq, D] */
  const void* dout;           /* upstream gradient [T, Hq, D] */
  const float* lse;           /* forward lse [Hq, T] */
  void* dq;                   /* [T, Hq, D]  */
  void* dk;                   /* [T, Hkv, D] */
  void* dv;                   /* [T, Hkv, D] */
  const int32_t* prefix_lens;
  const int32_t* causal_lens;
  const int32_t* cu_seqlens;
  int64_t q_stride_token, q_stride_head;
  int64_t k_stride_token, k_stride_head;
  int64_t v_stride_token, v_stride_head;
  int64_t out_stride_token, out_stride_head;
  int64_t dout_stride_token, dout_stride_head;
  int64_t dq_stride_token, dq_stride_head;
  int64_t dk_stride_token, dk_stride_head;
  int64_t dv_stride_token, dv_stride_head;
  int64_t lse_stride_head;
  int32_t total_tokens;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t numseqs;
  int32_t total_seqlen;
  int32_t max_seqlen_all;
  int32_t is_causal;
  int32_t dtype;
  float softmax_scale;
  void* workspace;            /* device memory, >= mimir_prefixlm_bwd_workspace_size(params) */
  size_t workspace_bytes;
  /* Optional sigmoid output gate (NULL: none), the backward of
   * gated_out = sigmoid(gate) * out.  With a gate, `dout` is the gradient of
   * gated_out and `out` the ungated attention output; the DELTA stage forms the
   * attention's upstream gradient round(dout * s) in the workspace, delta from
   * it, and dgate = round(round(dout * out) * (1 - s) * s) with s =
   * round(sigmoid(gate)), in the order torch's autograd evaluates the reference
   * expression (layers.py:239; sigmoid_backward = grad * (1 - y) * y). */
  const void* gate;           /* [T, Hq, D] */
  int64_t gate_stride_token, gate_stride_head;
  void* dgate;                /* [T, Hq, D]; required with a gate */
  int64_t dgate_stride_token, dgate_stride_head;
  /* Score-gradient hand-off (bf16, head_dim 128; no reference counterpart): when
   * the bf16 dS tiles of every (q head, 32-query block, 32-key block) fit in
   * this many bytes of workspace (mimir_prefixlm_bwd_dscore_bytes), the DKDV
   * stage writes them there and the DQ stage computes dQ = dS K from them
   * instead of recomputing S and dP; DQ then reads what DKDV wrote and runs
   * after it.  0: DQ recomputes.  The stored tiles carry no low half, so when
   * dS is split (split_mode) the recomputing dQ kernel runs instead: for ALWAYS
   * the hand-off is off, for AUTO both dQ kernels are enqueued and the one the
   * device-side decision selects does the work (the other exits at once).  The
   * recompute also takes over when a stored tile would fall outside the region
   * (a sequence longer than max_seqlen_all). */
  size_t dscore_limit_bytes;
  /* Low half of the forward output (NULL: delta from out alone; with split_flag
   * read only when the flag is set); see MimirPrefixLMFwdParams.out_lo. */
  const void* out_lo;         /* [T, Hq, D] */
  int64_t out_lo_stride_token, out_lo_stride_head;
  int32_t split_mode;         /* enum MimirSplitMode (bf16; dS in dK = dS^T Q and dQ = dS K) */
  const int32_t* split_flag;  /* the forward's recorded decision (device int32 [1]) or NULL */
  /* Optional gradient of a rotary position embedding inside the kernels (bf16
   * only; rope_cos NULL: none): q and k are the rotated operands the forward
   * used, and dq / dk receive the gradients of the unrotated q / k -- the bf16
   * gradient of the rotated operand mapped back in the kernels' stores exactly
   * as mimir_prefixlm_rope with inverse = 1 maps it (what autograd does for
   * layers.py:186-189).  Same tables as MimirPrefixLMFwdParams.rope_cos. */
  const float* rope_cos;
  const float* rope_sin;
  int64_t rope_stride_token;
  /* Key-range parts of the DQ stage (bf16; no reference counterpart): non-zero
   * lets mimir_prefixlm_bwd_workspace_size include, where the grid can be small
   * (ceil(total_tokens / 128) * num_q_heads < 512), a copy of the dQ tile list
   * with room for parts, arrival counters and 1024 / num_q_heads partial slots
   * of (4 * head_dim * 128 + 2048) bytes per q head; with a workspace that
   * large the dQ kernels cut the key ranges of their heaviest query tiles into
   * up to 16 parts run as separate workgroups, and the last part of a tile to
   * arrive sums the parts in part order (deterministic) and stores dQ.  0: no
   * parts. */
  int32_t dq_key_chunks;
} MimirPrefixLMBwdParams;

/* Bytes of device workspace the forward needs: the heaviest-first tile work list
 * (16-byte entries, one per 128-row query tile of every sequence; sized
 * ceil(T / 128) + numseqs, which bounds the tiles of any packing of T tokens into
 * numseqs sequences, so it does not rely on max_seqlen_all), then, 256-byte
 * aligned, the 512 int32 slots of the K scan behind split_mode AUTO. */
size_t mimir_prefixlm_fwd_workspace_bytes(int32_t total_tokens, int32_t numseqs, int32_t max_seqlen_all);

/* Bytes of device workspace with which the bf16 forward may also cut the key
 * ranges of its heaviest query tiles into parts (at most 16 per tile), run
 * them as separate workgroups and merge their partial outputs in part order
 * (deterministic): on a small grid -- fewer than 512 (query tile, q head)
 * workgroups -- the heaviest tiles otherwise run alone on a few compute units
 * at the end.  No counterpart in the reference (an extension of the forward's
 * own scheduling).  It adds 1024 / num_q_heads chunk slots of
 * (4 * head_dim * 128 + 2048) bytes per q head and their arrival counters; it
 * equals mimir_prefixlm_fwd_workspace_bytes where the grid cannot be small
 * (ceil(min(total_tokens, total_seqlen) / 128) * num_q_heads >= 512: the
 * least number of query tiles when cu_seqlens[0] = 0, as the reference's
 * metadata has it; with leading padding rows the grid can be smaller and then
 * runs uncut) and for float32.  The forward cuts key ranges iff its
 * workspace_bytes reaches this size; any size from
 * mimir_prefixlm_fwd_workspace_bytes up is valid.  Reads only dtype,
 * total_tokens, total_seqlen, num_q_heads, head_dim, numseqs and
 * max_seqlen_all. */
size_t mimir_prefixlm_fwd_workspace_size(const MimirPrefixLMFwdParams* params);

/* Forward: out (and lse if non-NULL).
 * Replaces the FA4 two-pass forward, src/mimir/model/flash_attention_prefixlm_fa4.py:353-406
 * (+ _fa4_varlen, fa4.py:17-50), the FA3 forward custom op
 * src/mimir/model/flash_attention_prefixlm_v2.py:101-144, and the masked-SDPA loop
 * src/mimir/model/flash_attention_prefixlm_dense.py:19-81. */
int mimir_prefixlm_fwd(const MimirPrefixLMFwdParams* params, void* stream);

/* The forward for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  It ignores params->workspace and keeps its
 * work list and K-scan slots in a fixed device array of 128 KiB inside the
 * library (one per GPU, held until the process ends): a call whose
 * mimir_prefixlm_fwd_workspace_bytes exceeds 128 KiB fails with
 * MIMIR_ERR_UNSUPPORTED_SHAPE before any device work (it fits while
 * ceil(total_tokens / 128) + numseqs <= 8064); it never cuts key ranges.  It calls no hipMalloc / hipFree.  Every call on one GPU
 * shares that array, so calls that overlap on one GPU (two streams or threads)
 * race; the array needs no clearing between calls.  The array's device address
 * is looked up once per device (the first call there) and kept: do not call it
 * after a hipDeviceReset (or another re-creation of the device's primary
 * context) in the same process.  Outputs as mimir_prefixlm_fwd. */
int mimir_prefixlm_fwd_noalloc(const MimirPrefixLMFwdParams* params, void* stream);

/* Backward: dq, dk, dv from dout, out and lse.  Deterministic: every gradient
 * element is summed in a fixed order by one owner (atomics only count work-queue
 * units and split-tile arrivals).
 * Replaces the FA3 backward custom op src/mimir/model/flash_attention_prefixlm_v2.py:165-227,
 * FA4's backward reached through fa4.py:153-179,309-331, and the Metal split
 * backward src/mimir/model/flash_attention_prefixlm_mps.py:1456-1561. */
int mimir_prefixlm_bwd(const MimirPrefixLMBwdParams* params, void* stream);

/* Backward stages, for callers that schedule them themselves (e.g. dK/dV and
 * dQ on two streams once delta is done).  mimir_prefixlm_bwd runs them all, in
 * order.  DELTA must complete before DKDV and DQ; DKDV, DQ and FILL are
 * independent of each other, except that with the score-gradient hand-off
 * (mimir_prefixlm_bwd_dscore_bytes non-zero) DQ reads what DKDV wrote.  No reference counterpart: the reference exposes
 * the backward only through autograd (flash_attention_prefixlm_v2.py:270-283). */
enum MimirBwdStage {
  MIMIR_BWD_STAGE_DELTA = 1, /* delta = rowsum(O * dO), lse * log2(e) and the tile work lists into the workspace */
  MIMIR_BWD_STAGE_DKDV = 2,  /* dK, dV for every key row inside a sequence */
  MIMIR_BWD_STAGE_DQ = 4,    /* dQ for every active query row */
  MIMIR_BWD_STAGE_FILL = 8,  /* zero dQ / dK / dV rows outside every sequence */
  MIMIR_BWD_STAGE_ALL = 15
};
int mimir_prefixlm_bwd_stages(const MimirPrefixLMBwdParams* params, int stages, void* stream);

/* Bytes of device workspace the backward needs: float32 delta = rowsum(O * dO) [Hq, T],
 * float32 lse * log2(e) [Hq, T], the tile work lists of the DQ and DKDV stages,
 * and for head_dim 128 the counters and float32 partial-sum slots of key tiles
 * that the DKDV stage splits in two (at most 384 (tile, kv head) splits, 256 KiB
 * each).  The DELTA stage writes the lists and zeroes the counters; DQ and DKDV
 * read them, and DKDV leaves the counters at zero. */
size_t mimir_prefixlm_bwd_workspace_bytes(int32_t total_tokens, int32_t num_q_heads, int32_t numseqs,
                                          int32_t max_seqlen_all);

/* Bytes of backward workspace for these parameters: mimir_prefixlm_bwd_workspace_bytes
 * plus, with a gate, the attention's upstream gradient [T, Hq, D] in the element type,
 * plus the score-gradient tiles when mimir_prefixlm_bwd_dscore_bytes(params) is non-zero,
 * plus the DQ stage's key-range parts when dq_key_chunks asks for them and the grid can
 * be small (the test of mimir_prefixlm_fwd_workspace_size).  Only the size fields
 * (total_tokens, total_seqlen, num_q_heads, numseqs, max_seqlen_all), head_dim,
 * dtype, gate, dscore_limit_bytes and dq_key_chunks are read. */
size_t mimir_prefixlm_bwd_workspace_size(const MimirPrefixLMBwdParams* params);

/* Bytes of workspace the score-gradient hand-off takes for these parameters, 0
 * when it is off: bf16 with head_dim 128 only, and only when the bf16 tiles,
 * Hq x (floor(T / 32) + numseqs + 1) x ceil(max_seqlen_all / 32) blocks of
 * 32 x 32, fit in dscore_limit_bytes.  No reference counterpart. */
size_t mimir_prefixlm_bwd_dscore_bytes(const MimirPrefixLMBwdParams* params);

/* Rotary position embedding on [T, H, D] rows, rotate-half convention
 * (reference: src/mimir/model/layers.py:24-40, apply_rotary_pos_emb on the q / k
 * splits of the fused projection, layers.py:183-189), cos / sin float32 [T, D]:
 *
 *   inverse == 0:  y = round(x * cos + rotate_half(x) * sin)   (fp32 math, one rounding)
 *   inverse != 0:  the gradient of that map, x_grad from y_grad, rounded as torch's
 *                  autograd does for the reference expression: each of the two
 *                  contributions (y_grad * cos and the rotate_half part of
 *                  y_grad * sin) is rounded to the element type, then their sum.
 *
 * rotate_half(x) = cat(-x[D/2:], x[:D/2]).  y may alias x (same pointer and
 * strides): every element pair is read before it is written.  bf16 needs
 * D % 16 == 0, float32 D % 8 == 0; rows 16-byte aligned. */
typedef struct MimirRopeParams {
  const void* x;              /* [T, H, D] */
  void* y;                    /* [T, H, D] */
  const float* cos;           /* [T, D] float32 */
  const float* sin;           /* [T, D] float32 */
  int64_t x_stride_token, x_stride_head;
  int64_t y_stride_token, y_stride_head;
  int64_t cs_stride_token;    /* cos / sin row stride (elements) */
  int32_t total_tokens;       /* T */
  int32_t num_heads;          /* H */
  int32_t head_dim;           /* D */
  int32_t dtype;              /* enum MimirDType */
  int32_t inverse;
} MimirRopeParams;
int mimir_prefixlm_rope(const MimirRopeParams* params, void* stream);

/* Attention against a static KV cache, the inference path of Mimir2's
 * Attention (reference: src/mimir/model/layers.py:134-167, _attention_with_cache,
 * with the Cache of layers.py:107-115).  For batch row b (cache row
 * r = batch_indices ? batch_indices[b] : b) and c = cache_lengths[b]:
 *
 *   1. k_new / v_new [b, i] are written to cache_k / cache_v [r, c + i], i < S;
 *   2. query i of q [b, i, h] attends the cache keys j < c + S of kv head
 *      h / (Hq / Hkv), and if `causal` only j <= c + i (the reference's mask);
 *      softmax scale `softmax_scale`, out [b, i, h] in the element type.
 *
 * c + S must not exceed cache_len (the reference raises IndexError there; this
 * entry point skips the cache writes and keys beyond the cache instead), and a
 * batch row whose cache row lies outside [0, cache_rows) gets a zero output and
 * no cache write (the reference raises IndexError).
 * max_kv_len is an upper bound of max_b(c + S) (the reference's
 * kv_len.max().item(), layers.py:143) that sizes the key split; each batch
 * row's own key range is split evenly over it.  bf16 only, head_dim 64 or 128.
 * The workspace holds the split partial results and one arrival counter per
 * (batch row, kv head, 128-row tile), which the call clears itself (no memset:
 * the call can be captured in a graph). */
typedef struct MimirCacheAttnParams {
  const void* q;              /* [B, S, Hq, D] */
  const void* k_new;          /* [B, S, Hkv, D] */
  const void* v_new;          /* [B, S, Hkv, D] */
  void* cache_k;              /* [>= rows, cache_len, Hkv, D] */
  void* cache_v;              /* [>= rows, cache_len, Hkv, D] */
  void* out;                  /* [B, S, Hq, D] */
  const void* cache_lengths;   /* device int32 or int64 [B] (index_int64) */
  const void* batch_indices;   /* device int32 or int64 [B], or NULL (row b) */
  int64_t q_stride_batch, q_stride_token, q_stride_head;
  int64_t kn_stride_batch, kn_stride_token, kn_stride_head;
  int64_t vn_stride_batch, vn_stride_token, vn_stride_head;
  int64_t ck_stride_batch, ck_stride_token, ck_stride_head;
  int64_t cv_stride_batch, cv_stride_token, cv_stride_head;
  int64_t out_stride_batch, out_stride_token, out_stride_head;
  int32_t batch;              /* B */
  int32_t seqlen;             /* S (1 for decode) */
  int32_t cache_len;          /* positions per cache row */
  int32_t cache_rows;         /* rows of cache_k / cache_v; rows outside [0, cache_rows) are skipped */
  int32_t max_kv_len;         /* upper bound of max_b(cache_lengths[b] + S) */
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t causal;
  int32_t dtype;              /* MIMIR_DTYPE_BFLOAT16 */
  float softmax_scale;
  void* workspace;            /* >= mimir_prefixlm_cache_attn_workspace_bytes(params) */
  size_t workspace_bytes;
  int32_t index_int64;        /* 1: cache_lengths / batch_indices are int64, 0: int32 */
} MimirCacheAttnParams;
size_t mimir_prefixlm_cache_attn_workspace_bytes(const MimirCacheAttnParams* params);
int mimir_prefixlm_cache_attn(const MimirCacheAttnParams* params, void* stream);

/* Device-side metadata check: writes to bad[0] (device int32 [2]) the first s in
 * [0, numseqs) whose lengths are invalid, or -1 if none, and to bad[1] why:
 *   1  prefix_lens[s] + causal_lens[s] != cu_seqlens[s+1] - cu_seqlens[s], or a
 *      negative length (the reference raises ValueError for this,
 *      src/mimir/model/flash_attention_prefixlm_dense.py:54-55);
 *   2  cu_seqlens[s+1] - cu_seqlens[s] > max_seqlen_all (the scalar sizes the
 *      score-gradient region and the per-sequence span check).
 * Asynchronous. */
int mimir_prefixlm_check_metadata(const int32_t* prefix_lens, const int32_t* causal_lens,
                                  const int32_t* cu_seqlens, int32_t numseqs, int32_t max_seqlen_all,
                                  int32_t* bad, void* stream);

/* Thread-local description of the last failure on this thread ("" if none). */
const char* mimir_prefixlm_last_error(void);

/* MIMIR_PREFIXLM_ABI_VERSION of the loaded library. */
int mimir_prefixlm_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MIMIR_PREFIXLM_H */
