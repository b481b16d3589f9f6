// C ABI of libmimir_prefixlm.so: argument validation, dtype / head_dim dispatch,
// padding-row fills and the metadata check.  Declarations and the contract live
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

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return MIMIR_OK;
  return fail(MIMIR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Rows that belong to no sequence, or lie at/after total_seqlen, are outputs of
// the operator too: O = 0, lse = -inf, dQ = 0 (flash_attention_prefixlm_dense.py:43,79-80).
// dK/dV rows outside every sequence are 0; key rows inside a sequence are written
// by the dK/dV kernel even at/after total_seqlen, since they remain keys there.
constexpr int kFillRows = 16;

struct FillArgs {
  void* x;            // [T, H, D] of elem_bytes
  int64_t st, sh;     // strides in elements
  float* lse;         // optional [H, T]
  int64_t lse_sh;
  const int32_t* cu_seqlens;
  int numseqs, total_seqlen, T, H, row_bytes, elem_bytes;
};

__global__ __launch_bounds__(256) void fill_rows_kernel(const FillArgs a) {
  const int t0 = blockIdx.x * kFillRows;
  const int first = a.numseqs > 0 ? a.cu_seqlens[0] : a.T;
  int last = a.numseqs > 0 ? a.cu_seqlens[a.numseqs] : 0;
  if (last > a.total_seqlen) last = a.total_seqlen;
  // inactive rows: t < first or t >= last
  const int t1 = min(t0 + kFillRows, a.T);
  if (t0 >= first && t1 <= last) return;
  const int chunks = a.row_bytes / 4;  // row_bytes is a multiple of 4
  for (int i = threadIdx.x; i < kFillRows * a.H * chunks; i += blockDim.x) {
    const int tt = i / (a.H * chunks);
    const int rem = i % (a.H * chunks);
    const int h = rem / chunks, c = rem % chunks;
    const int t = t0 + tt;
    if (t >= a.T || (t >= first && t < last)) continue;
    char* row = (char*)a.x + ((int64_t)t * a.st + (int64_t)h * a.sh) * a.elem_bytes;
    ((uint32_t*)row)[c] = 0u;
    if (c == 0 && a.lse != nullptr) a.lse[(int64_t)h * a.lse_sh + t] = -INFINITY;
  }
}

hipError_t launch_fill(void* x, int64_t st, int64_t sh, float* lse, int64_t lse_sh, const int32_t* cu,
                       int numseqs, int total_seqlen, int T, int H, int D, int elem_bytes,
                       hipStream_t stream) {
  if (T <= 0 || H <= 0) return hipSuccess;
  FillArgs a;
  a.x = x; a.st = st; a.sh = sh; a.lse = lse; a.lse_sh = lse_sh; a.cu_seqlens = cu;
  a.numseqs = numseqs; a.total_seqlen = total_seqlen; a.T = T; a.H = H;
  a.row_bytes = D * elem_bytes; a.elem_bytes = elem_bytes;
  hipLaunchKernelGGL(fill_rows_kernel, dim3((T + kFillRows - 1) / kFillRows), dim3(256), 0, stream, a);
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void check_metadata_kernel(const int32_t* prefix_lens,
                                                              const int32_t* causal_lens,
                                                              const int32_t* cu_seqlens, int numseqs,
                                                              int32_t* bad_seq) {
  __shared__ int best;
  if (threadIdx.x == 0) best = 0x7fffffff;
  __syncthreads();
  int mine = 0x7fffffff;
  for (int s = threadIdx.x; s < numseqs; s += blockDim.x) {
    const int len = cu_seqlens[s + 1] - cu_seqlens[s];
    const int p = prefix_lens[s], c = causal_lens[s];
    if (len < 0 || p < 0 || c < 0 || p + c != len) { mine = s; break; }
  }
  atomicMin(&best, mine);
  __syncthreads();
  if (threadIdx.x == 0) *bad_seq = best == 0x7fffffff ? -1 : best;
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

}  // namespace

extern "C" {

const char* mimir_prefixlm_last_error(void) { return g_last_error.c_str(); }

int mimir_prefixlm_abi_version(void) { return MIMIR_PREFIXLM_ABI_VERSION; }

size_t mimir_prefixlm_fwd_workspace_bytes(int32_t total_tokens, int32_t numseqs, int32_t max_seqlen_all) {
  if (total_tokens <= 0) return 0;
  return (size_t)mimir::plan_capacity(total_tokens, numseqs, max_seqlen_all) * sizeof(int2);
}

size_t mimir_prefixlm_bwd_workspace_bytes(int32_t total_tokens, int32_t num_q_heads, int32_t numseqs,
                                          int32_t max_seqlen_all) {
  if (total_tokens <= 0 || num_q_heads <= 0) return 0;
  // float32 delta [Hq, T], float32 lse * log2(e) [Hq, T], then the dQ and dK/dV tile lists
  return 2 * (size_t)total_tokens * (size_t)num_q_heads * sizeof(float) +
         2 * (size_t)mimir::plan_capacity(total_tokens, numseqs, max_seqlen_all) * sizeof(int2);
}

int mimir_prefixlm_check_metadata(const int32_t* prefix_lens, const int32_t* causal_lens,
                                  const int32_t* cu_seqlens, int32_t numseqs, int32_t* bad_seq,
                                  void* stream) {
  g_last_error.clear();
  if (bad_seq == nullptr) return fail(MIMIR_ERR_INVALID_ARGUMENT, "bad_seq is NULL");
  if (numseqs < 0) return fail(MIMIR_ERR_INVALID_ARGUMENT, "negative numseqs");
  if (numseqs > 0 && (prefix_lens == nullptr || causal_lens == nullptr || cu_seqlens == nullptr))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "metadata pointer is NULL");
  hipLaunchKernelGGL(check_metadata_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, prefix_lens,
                     causal_lens, cu_seqlens, numseqs, bad_seq);
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
  hipError_t e = dt == MIMIR_DTYPE_BFLOAT16 ? mimir_launch_fwd_bf16(*p, stream) : mimir_launch_fwd_f32(*p, stream);
  if ((rc = hip_status(e, "forward launch"))) return rc;
  e = launch_fill(p->out, p->out_stride_token, p->out_stride_head, p->lse, p->lse_stride_head, p->cu_seqlens,
                  p->numseqs, p->total_seqlen, p->total_tokens, p->num_q_heads, D, elem_bytes_of(dt), stream);
  return hip_status(e, "forward padding fill");
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
  const size_t need =
      mimir_prefixlm_bwd_workspace_bytes(p->total_tokens, p->num_q_heads, p->numseqs, p->max_seqlen_all);
  if (p->workspace == nullptr || p->workspace_bytes < need || !aligned16(p->workspace))
    return fail(MIMIR_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned and hold at least " +
                                                std::to_string(need) + " bytes");
  hipError_t e = dt == MIMIR_DTYPE_BFLOAT16 ? mimir_launch_bwd_bf16(*p, stream, stages)
                                            : mimir_launch_bwd_f32(*p, stream, stages);
  if ((rc = hip_status(e, "backward launch"))) return rc;
  if (!(stages & MIMIR_BWD_STAGE_FILL)) return MIMIR_OK;
  const int es = elem_bytes_of(dt);
  e = launch_fill(p->dq, p->dq_stride_token, p->dq_stride_head, nullptr, 0, p->cu_seqlens, p->numseqs,
                  p->total_seqlen, p->total_tokens, p->num_q_heads, D, es, stream);
  if ((rc = hip_status(e, "dq padding fill"))) return rc;
  e = launch_fill(p->dk, p->dk_stride_token, p->dk_stride_head, nullptr, 0, p->cu_seqlens, p->numseqs,
                  p->total_tokens, p->total_tokens, p->num_kv_heads, D, es, stream);
  if ((rc = hip_status(e, "dk padding fill"))) return rc;
  e = launch_fill(p->dv, p->dv_stride_token, p->dv_stride_head, nullptr, 0, p->cu_seqlens, p->numseqs,
                  p->total_tokens, p->total_tokens, p->num_kv_heads, D, es, stream);
  return hip_status(e, "dv padding fill");
}

}  // extern "C"
