// C ABI of libmimir_prefixlm.so: argument validation, dtype / head_dim dispatch
// and the metadata check.  Declarations and the contract live
// in include/mimir_prefixlm.h.
#include <cmath>
#include <cstdio>
#include <string>

#include "prefixlm_common.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

}  // namespace

namespace mimir {
int fail_with(int code, const std::string& msg) { return fail(code, msg); }
}  // namespace mimir

namespace {

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MIMIR_OK;
  return fail(MIMIR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// bad[0]: the first invalid sequence (-1: none); bad[1]: 1 for inconsistent or
// negative lengths, 2 for a length above max_seqlen_all.
__global__ __launch_bounds__(256) void check_metadata_kernel(const int32_t* prefix_lens,
                                                              const int32_t* causal_lens,
                                                              const int32_t* cu_seqlens, int numseqs,
                                                              int max_seqlen_all, int32_t* bad) {
  __shared__ int best;
  if (threadIdx.x == 0) best = 0x7fffffff;
  __syncthreads();
  int mine = 0x7fffffff;
  for (int s = threadIdx.x; s < numseqs; s += blockDim.x) {
    const int len = cu_seqlens[s + 1] - cu_seqlens[s];
    const int p = prefix_lens[s], c = causal_lens[s];
    if (len < 0 || p < 0 || c < 0 || p + c != len || len > max_seqlen_all) { mine = s; break; }
  }
  atomicMin(&best, mine);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int s = best == 0x7fffffff ? -1 : best;
    int why = 0;
    if (s >= 0) {
      const int len = cu_seqlens[s + 1] - cu_seqlens[s];
      const int p = prefix_lens[s], c = causal_lens[s];
      why = (len < 0 || p < 0 || c < 0 || p + c != len) ? 1 : 2;
    }
    bad[0] = s;
    bad[1] = why;
  }
}

int elem_bytes_of(int dtype) { return dtype == MIMIR_DTYPE_FLOAT32 ? 4 : 2; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Common checks of the forward / backward geometry.
int check_common(int dtype, int T, int Hq, int Hkv, int D, int numseqs, int total_seqlen,
                 int max_seqlen_all, float scale) {
  if (dtype != MIMIR_DTYPE_FLOAT32 && dtype != MIMIR_DTYPE_BFLOAT16)
    return fail(MIMIR_ERR_UNSUPPORTED_DTYPE,
                "prefix-LM attention supports float32 and bfloat16 tensors only (dtype code " +
                    std::to_string(dtype) + ")");
  if (T < 0 || numseqs < 0 || total_seqlen < 0 || max_seqlen_all < 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "negative size argument");
  if (Hq <= 0 || Hkv <= 0 || D <= 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "head counts and head_dim must be positive");
  if (Hq % Hkv != 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "Query heads " + std::to_string(Hq) +
                                                " must be divisible by key/value heads " + std::to_string(Hkv) + ".");
  if (total_seqlen > T)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "total_seqlen " + std::to_string(total_seqlen) +
                                                " exceeds the packed length " + std::to_string(T));
  if (numseqs > T + 1 && T > 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "numseqs exceeds the metadata length");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "softmax_scale must be positive and finite");
  const bool ok_d = dtype == MIMIR_DTYPE_BFLOAT16 ? mimir_bf16_head_dim_supported(D) : mimir_f32_head_dim_supported(D);
  if (!ok_d)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE,
                std::string("head_dim ") + std::to_string(D) + " is not supported for " +
                    (dtype == MIMIR_DTYPE_BFLOAT16 ? "bfloat16 (supported: 64, 128)" : "float32 (supported: 32, 64, 96, 128)"));
  return MIMIR_OK;
}

// A tensor operand: data pointer plus token / head strides (elements).
int check_operand(const char* name, const void* ptr, int64_t st, int64_t sh, int D, int dtype, int max_rows) {
  if (ptr == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, std::string(name) + " is NULL");
  const int vec = dtype == MIMIR_DTYPE_FLOAT32 ? 4 : 8;  // elements per 16-byte access
  if (!aligned16(ptr) || st % vec != 0 || sh % vec != 0)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE,
                std::string(name) + " must be 16-byte aligned with token/head strides that are multiples of " +
                    std::to_string(vec) + " elements");
  if (st < D || sh < 0) return fail(MIMIR_ERR_UNSUPPORTED_SHAPE, std::string(name) + " rows overlap (token stride < head_dim)");
  // Per-sequence byte offsets are 32-bit inside the kernels.
  const double span = ((double)max_rows + 256.0) * (double)st * (double)elem_bytes_of(dtype);
  if (span >= 2147483648.0)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE,
                std::string(name) + ": a sequence spans more than 2 GiB; split the batch");
  return MIMIR_OK;
}

// RoPE tables of the fused rotation (bf16 kernels only).
int check_rope(int dtype, int D, const float* cos, const float* sin, int64_t st) {
  if (cos == nullptr && sin == nullptr) return MIMIR_OK;
  if (dtype != MIMIR_DTYPE_BFLOAT16)
    return fail(MIMIR_ERR_UNSUPPORTED_DTYPE, "RoPE inside the attention kernels is bfloat16 only; for float32 "
                                             "rotate with mimir_prefixlm_rope");
  if (cos == nullptr || sin == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "rope_cos and rope_sin go together");
  if (!aligned16(cos) || !aligned16(sin) || st % 4 != 0 || st < D)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "rope_cos / rope_sin rows must be 16-byte aligned float32 rows of at "
                                            "least head_dim elements (rope_stride_token a multiple of 4)");
  return MIMIR_OK;
}

}  // namespace

extern "C" {

const char* mimir_prefixlm_last_error(void) { return g_last_error.c_str(); }

int mimir_prefixlm_abi_version(void) { return MIMIR_PREFIXLM_ABI_VERSION; }

size_t mimir_prefixlm_fwd_workspace_bytes(int32_t total_tokens, int32_t numseqs, int32_t max_seqlen_all) {
  const int cap = mimir::plan_capacity(total_tokens, numseqs, max_seqlen_all);
  if (cap <= 0) return 0;
  return mimir::fwd_workspace_layout(cap, 0, 0, false).total;
}

size_t mimir_prefixlm_fwd_workspace_size(const MimirPrefixLMFwdParams* p) {
  if (p == nullptr) return 0;
  const size_t base = mimir_prefixlm_fwd_workspace_bytes(p->total_tokens, p->numseqs, p->max_seqlen_all);
  // key-range parts: bf16 only, and only where the grid can be small (a list of
  // at least ceil(min(T, total_seqlen) / 128) query tiles per q head fills
  // kChunkWgs otherwise)
  if (base == 0 || p->dtype != MIMIR_DTYPE_BFLOAT16 || p->head_dim <= 0 ||
      !mimir::chunk_grid_can_be_small(p->total_tokens, p->total_seqlen, p->num_q_heads))
    return base;
  const int cap = mimir::plan_capacity(p->total_tokens, p->numseqs, p->max_seqlen_all);
  return mimir::fwd_workspace_layout(cap, p->num_q_heads, p->head_dim, true).total;
}

size_t mimir_prefixlm_bwd_dscore_bytes(const MimirPrefixLMBwdParams* p) {
  // the stored tiles have no low half: no hand-off when dS is always split
  if (p == nullptr || p->dtype != MIMIR_DTYPE_BFLOAT16 || p->head_dim != 128 || p->total_tokens <= 0 ||
      p->num_q_heads <= 0 || p->dscore_limit_bytes == 0 || p->split_mode == MIMIR_SPLIT_ALWAYS)
    return 0;
  const mimir::DscoreGeom g = mimir::dscore_geometry(p->total_tokens, p->num_q_heads, p->numseqs, p->max_seqlen_all);
  return g.bytes <= p->dscore_limit_bytes ? g.bytes : 0;
}

size_t mimir_prefixlm_bwd_workspace_size(const MimirPrefixLMBwdParams* p) {
  if (p == nullptr || p->total_tokens <= 0 || p->num_q_heads <= 0) return 0;
  const size_t dout_bytes = p->gate != nullptr ? (size_t)p->total_tokens * (size_t)p->num_q_heads *
                                                     (size_t)(p->head_dim > 0 ? p->head_dim : 0) *
                                                     (size_t)elem_bytes_of(p->dtype)
                                               : 0;
  return mimir::bwd_workspace_layout(p->total_tokens, p->num_q_heads, p->numseqs, p->max_seqlen_all, dout_bytes,
                                     mimir_prefixlm_bwd_dscore_bytes(p), mimir::bwd_chunk_head_dim(*p))
      .total;
}

size_t mimir_prefixlm_bwd_workspace_bytes(int32_t total_tokens, int32_t num_q_heads, int32_t numseqs,
                                          int32_t max_seqlen_all) {
  if (total_tokens <= 0 || num_q_heads <= 0) return 0;
  // float32 delta [Hq, T], float32 lse * log2(e) [Hq, T], the dQ and dK/dV tile
  // lists, the split counters and the split dK/dV partial slots
  return mimir::bwd_workspace_layout(total_tokens, num_q_heads, numseqs, max_seqlen_all).total;
}

int mimir_prefixlm_check_metadata(const int32_t* prefix_lens, const int32_t* causal_lens,
                                  const int32_t* cu_seqlens, int32_t numseqs, int32_t max_seqlen_all,
                                  int32_t* bad, void* stream) {
  g_last_error.clear();
  if (bad == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "bad is NULL");
  if (numseqs < 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "negative numseqs");
  if (numseqs > 0 && (prefix_lens == nullptr || causal_lens == nullptr || cu_seqlens == nullptr))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "metadata pointer is NULL");
  hipLaunchKernelGGL(check_metadata_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, prefix_lens,
                     causal_lens, cu_seqlens, numseqs, max_seqlen_all, bad);
  return hip_status(hipGetLastError(), "metadata check launch");
}

int mimir_prefixlm_fwd(const MimirPrefixLMFwdParams* p, void* stream_) {
  g_last_error.clear();
  if (p == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "params is NULL");
  hipStream_t stream = (hipStream_t)stream_;
  int rc = check_common(p->dtype, p->total_tokens, p->num_q_heads, p->num_kv_heads, p->head_dim, p->numseqs,
                        p->total_seqlen, p->max_seqlen_all, p->softmax_scale);
  if (rc) return rc;
  if (p->total_tokens == 0) return MIMIR_OK;
  const int D = p->head_dim, dt = p->dtype, rows = p->max_seqlen_all;
  if ((rc = check_operand("q", p->q, p->q_stride_token, p->q_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("k", p->k, p->k_stride_token, p->k_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("v", p->v, p->v_stride_token, p->v_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("out", p->out, p->out_stride_token, p->out_stride_head, D, dt, rows))) return rc;
  if (p->numseqs > 0 && (p->prefix_lens == nullptr || p->cu_seqlens == nullptr))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "metadata pointer is NULL");
  if (p->lse != nullptr && p->lse_stride_head < p->total_tokens)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "lse head stride is smaller than the packed length");
  const size_t need = mimir_prefixlm_fwd_workspace_bytes(p->total_tokens, p->numseqs, p->max_seqlen_all);
  if (need > 0 && (p->workspace == nullptr || p->workspace_bytes < need || !aligned16(p->workspace)))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned and hold at least " +
                                                std::to_string(need) + " bytes");
  if (p->gate != nullptr) {
    if ((rc = check_operand("gate", p->gate, p->gate_stride_token, p->gate_stride_head, D, dt, rows))) return rc;
    if ((rc = check_operand("gated_out", p->gated_out, p->gated_out_stride_token, p->gated_out_stride_head, D, dt,
                            rows)))
      return rc;
  }
  if (p->split_mode < MIMIR_SPLIT_AUTO || p->split_mode > MIMIR_SPLIT_NEVER)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "split_mode must be MIMIR_SPLIT_AUTO, _ALWAYS or _NEVER");
  if (((uintptr_t)p->split_flag & 3u) != 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "split_flag must be 4-byte aligned");
  if ((rc = check_rope(dt, D, p->rope_cos, p->rope_sin, p->rope_stride_token))) return rc;
  if (p->q_rope != nullptr) {
    if (p->rope_cos == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "q_rope needs rope_cos / rope_sin");
    if ((rc = check_operand("q_rope", p->q_rope, p->q_rope_stride_token, p->q_rope_stride_head, D, dt, rows)))
      return rc;
  }
  if (p->out_lo != nullptr) {
    if (dt != MIMIR_DTYPE_BFLOAT16)
      return fail(MIMIR_ERR_INVALID_ARGUMENT, "out_lo is a bfloat16 output (float32 needs no low half)");
    if ((rc = check_operand("out_lo", p->out_lo, p->out_lo_stride_token, p->out_lo_stride_head, D, dt, rows)))
      return rc;
  }
  mimir::Prologue pro;
  pro.fill[pro.nfill++] = mimir::fill_args(p->out, p->out_stride_token, p->out_stride_head, p->lse,
                                           p->lse_stride_head, p->cu_seqlens, p->numseqs, p->total_seqlen,
                                           p->total_tokens, p->num_q_heads, D, elem_bytes_of(dt));
  if (p->out_lo != nullptr)  // padding rows: O = 0 exactly, so its low half is 0
    pro.fill[pro.nfill++] = mimir::fill_args(p->out_lo, p->out_lo_stride_token, p->out_lo_stride_head, nullptr, 0,
                                             p->cu_seqlens, p->numseqs, p->total_seqlen, p->total_tokens,
                                             p->num_q_heads, D, elem_bytes_of(dt));
  hipError_t e;
  if (dt == MIMIR_DTYPE_BFLOAT16) {
    // gated_out rows outside the attended rows are sigmoid(gate) * 0 = 0
    if (p->gate != nullptr)
      pro.fill[pro.nfill++] = mimir::fill_args(p->gated_out, p->gated_out_stride_token, p->gated_out_stride_head,
                                               nullptr, 0, p->cu_seqlens, p->numseqs, p->total_seqlen,
                                               p->total_tokens, p->num_q_heads, D, elem_bytes_of(dt));
    e = mimir_launch_fwd_bf16(*p, pro, stream);
  } else {
    e = mimir::launch_prologue(pro, stream);
    if (e == hipSuccess) e = mimir_launch_fwd_f32(*p, stream);
    if (e == hipSuccess && p->gate != nullptr) e = mimir::launch_gate_fwd_f32(*p, stream);
  }
  return hip_status(e, "forward launch");
}

int mimir_prefixlm_bwd(const MimirPrefixLMBwdParams* p, void* stream) {
  return mimir_prefixlm_bwd_stages(p, MIMIR_BWD_STAGE_ALL, stream);
}

int mimir_prefixlm_bwd_stages(const MimirPrefixLMBwdParams* p, int stages, void* stream_) {
  g_last_error.clear();
  if (p == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "params is NULL");
  if (stages & ~MIMIR_BWD_STAGE_ALL) return fail(MIMIR_ERR_INVALID_ARGUMENT, "unknown backward stage bits");
  hipStream_t stream = (hipStream_t)stream_;
  int rc = check_common(p->dtype, p->total_tokens, p->num_q_heads, p->num_kv_heads, p->head_dim, p->numseqs,
                        p->total_seqlen, p->max_seqlen_all, p->softmax_scale);
  if (rc) return rc;
  if (p->total_tokens == 0) return MIMIR_OK;
  const int D = p->head_dim, dt = p->dtype, rows = p->max_seqlen_all;
  if ((rc = check_operand("q", p->q, p->q_stride_token, p->q_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("k", p->k, p->k_stride_token, p->k_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("v", p->v, p->v_stride_token, p->v_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("out", p->out, p->out_stride_token, p->out_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("dout", p->dout, p->dout_stride_token, p->dout_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("dq", p->dq, p->dq_stride_token, p->dq_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("dk", p->dk, p->dk_stride_token, p->dk_stride_head, D, dt, rows))) return rc;
  if ((rc = check_operand("dv", p->dv, p->dv_stride_token, p->dv_stride_head, D, dt, rows))) return rc;
  if (p->lse == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "lse is NULL");
  if (p->lse_stride_head < p->total_tokens)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "lse head stride is smaller than the packed length");
  if (p->numseqs > 0 && (p->prefix_lens == nullptr || p->cu_seqlens == nullptr))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "metadata pointer is NULL");
  if (p->gate != nullptr) {
    if ((rc = check_operand("gate", p->gate, p->gate_stride_token, p->gate_stride_head, D, dt, rows))) return rc;
    if ((rc = check_operand("dgate", p->dgate, p->dgate_stride_token, p->dgate_stride_head, D, dt, rows)))
      return rc;
  }
  if (p->out_lo != nullptr) {
    if (dt != MIMIR_DTYPE_BFLOAT16)
      return fail(MIMIR_ERR_INVALID_ARGUMENT, "out_lo is a bfloat16 input (float32 needs no low half)");
    if ((rc = check_operand("out_lo", p->out_lo, p->out_lo_stride_token, p->out_lo_stride_head, D, dt, rows)))
      return rc;
  }
  if (p->split_mode < MIMIR_SPLIT_AUTO || p->split_mode > MIMIR_SPLIT_NEVER)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "split_mode must be MIMIR_SPLIT_AUTO, _ALWAYS or _NEVER");
  if (((uintptr_t)p->split_flag & 3u) != 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "split_flag must be 4-byte aligned");
  if ((rc = check_rope(dt, D, p->rope_cos, p->rope_sin, p->rope_stride_token))) return rc;
  const size_t need = mimir_prefixlm_bwd_workspace_size(p);
  if (p->workspace == nullptr || p->workspace_bytes < need || !aligned16(p->workspace))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned and hold at least " +
                                                std::to_string(need) + " bytes");
  mimir::Prologue pro;
  if (stages & MIMIR_BWD_STAGE_FILL) {
    // dQ rows at/after total_seqlen are zero; dK / dV rows inside a sequence stay keys there.
    const int es = elem_bytes_of(dt);
    pro.fill[pro.nfill++] = mimir::fill_args(p->dq, p->dq_stride_token, p->dq_stride_head, nullptr, 0, p->cu_seqlens,
                                             p->numseqs, p->total_seqlen, p->total_tokens, p->num_q_heads, D, es);
    pro.fill[pro.nfill++] = mimir::fill_args(p->dk, p->dk_stride_token, p->dk_stride_head, nullptr, 0, p->cu_seqlens,
                                             p->numseqs, p->total_tokens, p->total_tokens, p->num_kv_heads, D, es);
    pro.fill[pro.nfill++] = mimir::fill_args(p->dv, p->dv_stride_token, p->dv_stride_head, nullptr, 0, p->cu_seqlens,
                                             p->numseqs, p->total_tokens, p->total_tokens, p->num_kv_heads, D, es);
  }
  hipError_t e;
  if (dt == MIMIR_DTYPE_BFLOAT16) {
    e = mimir_launch_bwd_bf16(*p, pro, stream, stages);
  } else if (p->gate == nullptr) {
    e = mimir::launch_prologue(pro, stream);
    if (e == hipSuccess) e = mimir_launch_bwd_f32(*p, stream, stages);
  } else {
    // float32 with a gate: the gate rows form the attention's upstream gradient and
    // delta in the workspace; the attention stages then read that gradient.
    const mimir::BwdWorkspace ws = mimir::bwd_workspace_layout(
        p->total_tokens, p->num_q_heads, p->numseqs, p->max_seqlen_all,
        (size_t)p->total_tokens * p->num_q_heads * D * sizeof(float));
    float* const dout_s = (float*)((char*)p->workspace + ws.dout);
    e = mimir::launch_prologue(pro, stream);
    if (e == hipSuccess && (stages & MIMIR_BWD_STAGE_DELTA))
      e = mimir::launch_gate_bwd_f32(*p, dout_s, (float*)((char*)p->workspace + ws.delta), stream);
    if (e == hipSuccess) {
      MimirPrefixLMBwdParams q = *p;
      q.dout = dout_s;
      q.dout_stride_token = (int64_t)p->num_q_heads * D;
      q.dout_stride_head = D;
      e = mimir_launch_bwd_f32(q, stream, stages & ~MIMIR_BWD_STAGE_DELTA);
    }
  }
  return hip_status(e, "backward launch");
}

size_t mimir_prefixlm_cache_attn_workspace_bytes(const MimirCacheAttnParams* p) {
  if (p == nullptr || p->batch <= 0 || p->seqlen <= 0 || p->num_kv_heads <= 0 || p->num_q_heads <= 0 ||
      p->cache_len <= 0)
    return 0;
  return mimir::cache_split(*p).workspace_bytes;
}

int mimir_prefixlm_cache_attn(const MimirCacheAttnParams* p, void* stream) {
  g_last_error.clear();
  if (p == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "params is NULL");
  if (p->dtype != MIMIR_DTYPE_BFLOAT16)
    return fail(MIMIR_ERR_UNSUPPORTED_DTYPE, "KV-cache attention supports bfloat16 tensors only (dtype code " +
                                                 std::to_string(p->dtype) + ")");
  if (p->batch < 0 || p->seqlen < 0 || p->cache_len < 0 || p->cache_rows < 0 || p->num_q_heads <= 0 ||
      p->num_kv_heads <= 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "negative size or non-positive head count");
  if (p->num_q_heads % p->num_kv_heads != 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "Query heads " + std::to_string(p->num_q_heads) +
                                                " must be divisible by key/value heads " +
                                                std::to_string(p->num_kv_heads) + ".");
  if (!mimir_bf16_head_dim_supported(p->head_dim))
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE, "head_dim " + std::to_string(p->head_dim) +
                                                 " is not supported for bfloat16 (supported: 64, 128)");
  if (!(p->softmax_scale > 0.f) || !std::isfinite(p->softmax_scale))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "softmax_scale must be positive and finite");
  if (p->batch == 0 || p->seqlen == 0) return MIMIR_OK;
  if (p->cache_len == 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "the cache holds no positions");
  if (p->cache_lengths == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "cache_lengths is NULL");
  const int D = p->head_dim, dt = p->dtype;
  int rc;
  // per batch row a [rows, H, D] tensor: the span checks of the packed operands apply per row
  if ((rc = check_operand("q", p->q, p->q_stride_token, p->q_stride_head, D, dt, p->seqlen))) return rc;
  if ((rc = check_operand("k_new", p->k_new, p->kn_stride_token, p->kn_stride_head, D, dt, p->seqlen))) return rc;
  if ((rc = check_operand("v_new", p->v_new, p->vn_stride_token, p->vn_stride_head, D, dt, p->seqlen))) return rc;
  if ((rc = check_operand("out", p->out, p->out_stride_token, p->out_stride_head, D, dt, p->seqlen))) return rc;
  if ((rc = check_operand("cache_k", p->cache_k, p->ck_stride_token, p->ck_stride_head, D, dt, p->cache_len)))
    return rc;
  if ((rc = check_operand("cache_v", p->cache_v, p->cv_stride_token, p->cv_stride_head, D, dt, p->cache_len)))
    return rc;
  const int64_t bs[6] = {p->q_stride_batch, p->kn_stride_batch, p->vn_stride_batch, p->ck_stride_batch,
                         p->cv_stride_batch, p->out_stride_batch};
  for (int64_t b : bs)
    if (b < 0 || b % 8 != 0)
      return fail(MIMIR_ERR_UNSUPPORTED_SHAPE, "batch strides must be non-negative multiples of 8 elements");
  const size_t need = mimir_prefixlm_cache_attn_workspace_bytes(p);
  if (need > 0 && (p->workspace == nullptr || p->workspace_bytes < need || !aligned16(p->workspace)))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned and hold at least " +
                                                std::to_string(need) + " bytes");
  return hip_status(mimir::launch_cache_attn_bf16(*p, (hipStream_t)stream), "KV-cache attention launch");
}

int mimir_prefixlm_rope(const MimirRopeParams* p, void* stream) {
  g_last_error.clear();
  if (p == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "params is NULL");
  if (p->dtype != MIMIR_DTYPE_FLOAT32 && p->dtype != MIMIR_DTYPE_BFLOAT16)
    return fail(MIMIR_ERR_UNSUPPORTED_DTYPE, "RoPE supports float32 and bfloat16 tensors only (dtype code " +
                                                 std::to_string(p->dtype) + ")");
  if (p->total_tokens < 0 || p->num_heads <= 0 || p->head_dim <= 0)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "negative size or non-positive heads / head_dim");
  const int vec = p->dtype == MIMIR_DTYPE_FLOAT32 ? 4 : 8;  // elements per 16-byte access
  if (p->head_dim % (2 * vec) != 0)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE, "RoPE head_dim " + std::to_string(p->head_dim) + " must be a multiple of " +
                                                 std::to_string(2 * vec) + " for this dtype");
  if (p->total_tokens == 0) return MIMIR_OK;
  if (p->x == nullptr || p->y == nullptr || p->cos == nullptr || p->sin == nullptr)
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "RoPE tensor pointer is NULL");
  if (!aligned16(p->x) || !aligned16(p->y) || !aligned16(p->cos) || !aligned16(p->sin) ||
      p->x_stride_token % vec || p->x_stride_head % vec || p->y_stride_token % vec || p->y_stride_head % vec ||
      p->cs_stride_token % 4)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE,
                "RoPE tensors must be 16-byte aligned with strides that are multiples of 16 bytes");
  if (p->cs_stride_token < p->head_dim || p->x_stride_head < 0 || p->y_stride_head < 0)
    return fail(MIMIR_ERR_UNSUPPORTED_SHAPE, "RoPE rows overlap");
  return hip_status(mimir::launch_rope(*p, (hipStream_t)stream), "RoPE launch");
}

}  // extern "C"
